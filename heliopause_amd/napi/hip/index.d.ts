// Types of hip/index.js: the "hip" runner provider, shaped like
// createWasmProvider (packages/engine/src/runner/wasm/index.ts:64-87) and
// ModelRunnerProvider (runner/provider.ts:30-36).
import type { HipProviderOptions, HipSession } from "./acceleration";

export * from "./acceleration";
export * from "./layers";
export * from "./segment-runner";

/* SegmentRunnerProvider (runner/segment-runner.ts:6) with the HIP member. */
export type SegmentRunnerProvider = "reference" | "wasm" | "webgpu" | "hip";

/* The engine pieces the provider builds on (ModelRunner, model-runner.ts:54-73,
 * and createModelResourceRequirements, model-resources.ts:58). */
export type HipEngine<TRunner extends { provider: string; segmentRunner(options: unknown): unknown }, TRequirements> = {
  createWasmModelRunner(): TRunner;
  createModelResourceRequirements(options: {
    provider: "hip";
    gguf: unknown;
    manifest: unknown;
    contextLength: number;
    slidingWindowReserveTokens?: number;
    memoryLimitBytes: number;
    targetResourceConstrained: boolean;
    canRunFullModel: boolean;
    plannedReason: string;
  }): TRequirements;
};

export const DEFAULT_HBM_BYTES: number;

export function createHipModelRunner<TRunner extends { provider: string; segmentRunner(options: unknown): unknown }>(
  engine: HipEngine<TRunner, unknown>,
): Omit<TRunner, "provider"> & { provider: "hip" };

export function createHipProvider<TRunner extends { provider: string; segmentRunner(options: unknown): unknown }, TRequirements>(
  options: HipProviderOptions | undefined,
  engine: HipEngine<TRunner, TRequirements>,
): {
  readonly name: "hip";
  readonly options: Readonly<HipProviderOptions>;
  createModelRunner(): Omit<TRunner, "provider"> & { provider: "hip" };
  modelResourceRequirements(
    session: HipSession & { manifest: unknown; tensorReader: { metadata: unknown } },
    options: { contextLength: number; slidingWindowReserveTokens?: number },
  ): TRequirements;
};
