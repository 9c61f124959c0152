// Types of hip/acceleration.js: the HIP execution provider's session state,
// shaped like packages/engine/src/runner/wasm/acceleration.ts.
import type { HipQuantizedWeightHandle, QuantizedType } from "../hip-kernels";

/* The members of ModelSession (runtime.ts) the provider uses. */
export type HipSession = {
  hasProvider(name: string): boolean;
  provider<T = { options: HipProviderOptions }>(name: string): T | undefined;
  setExecutionProviderStatsProvider(provider: () => Record<string, number | boolean>, name: string): void;
  getTensor(name: string): { name?: string; type: string; dimensions: readonly number[] };
  tensorReader: {
    readTensorBytes(name: string): Promise<Uint8Array>;
    metadata?: { tensors: ReadonlyArray<{ name: string }> };
  };
};

export type HipProviderOptions = {
  residentWeightCache?: boolean;
  projectionBatching?: boolean;
  memoryLimitBytes?: number;
};

export type HipExecutionProviderStats = {
  hipResidentWeightCacheEnabled: boolean;
  hipResidentWeightCacheCount: number;
  hipResidentWeightCacheBytes: number;
  hipResidentWeightCacheHits: number;
  hipResidentWeightCacheMisses: number;
  hipResidentWeightCacheDeclined: number;
};

export function registerHipExecutionProvider(session: HipSession): void;
export function hipExecutionProviderStats(session: HipSession): HipExecutionProviderStats;
export function shutdownHipExecutionProvider(session: HipSession): void;
export function hipExecutionProviderEnabled(session: HipSession): boolean;
export function hipResidentWeightCacheEnabled(session: HipSession): boolean;
export function hipProjectionBatchingEnabled(session: HipSession): boolean;
export function readHipWeightHandle(
  session: HipSession,
  name: string,
  type: QuantizedType,
  inputSize: number,
  rowCount: number,
): Promise<HipQuantizedWeightHandle | undefined>;
export function adoptHipWeightHandles(
  session: HipSession,
  handles: Map<string, HipQuantizedWeightHandle | undefined>,
): void;
export function setHipKernels(module: typeof import("../hip-kernels")): void;
export function hipKernels(): typeof import("../hip-kernels");
