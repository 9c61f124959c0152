// Types of hip/segment-runner.js: the device SegmentRunner
// (runner/segment-runner.ts:18-34) of the "hip" provider.
import type { ResolvedHipSamplingOptions } from "../hip-kernels";

export type HipInferenceState = {
  fullAttention: Map<number, {
    key: Float32Array; value: Float32Array; keyLength: number; valueLength: number; headCountKv: number;
    kind: "full" | "sliding"; contextLength: number; capacity: number;
  }>;
  contextLength: number;
  nextPosition: number;
};

export type HipSegmentRunOptions = { trace?: unknown; perLayerInputs?: Float32Array; attentionCausal?: boolean };

export declare class HipSegmentRunner {
  readonly provider: "hip";
  readonly segmentStartLayer: number;
  readonly segmentEndLayerExclusive: number;
  runTokensHidden(inputHidden: Float32Array, positions: Int32Array, state: HipInferenceState,
    options?: HipSegmentRunOptions): Promise<{ hidden: Float32Array }>;
  runTokenHidden(inputHidden: Float32Array, positions: Int32Array, state: HipInferenceState,
    options?: HipSegmentRunOptions): Promise<{ hidden: Float32Array }>;
  runToken(inputHidden: Float32Array, positions: Int32Array, state: HipInferenceState, options?: {
    topK?: number; sampling?: ResolvedHipSamplingOptions; samplingState?: Uint32Array;
  }): Promise<{ selectedTokenId?: number; topTokens: { id: number; value: number }[];
    distribution?: { id: number; value: number; probability: number }[] }>;
  release(): void;
}

export function createHipSegmentRunner(options: {
  session: unknown; state?: HipInferenceState; manifest?: unknown; epsilon?: number;
  segmentStartLayer?: number; segmentEndLayerExclusive?: number;
}): Promise<HipSegmentRunner | undefined>;
export function hipSegmentSupport(session: unknown, manifest: unknown, start: number, end: number):
  { supported: boolean; reason?: string };
export function f16Bits(value: number): number;
export function deviceRingFromHost(cache: HipInferenceState["fullAttention"] extends Map<number, infer C> ? C : never):
  { key: Uint16Array; value: Uint16Array };
