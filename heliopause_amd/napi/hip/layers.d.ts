// Types of hip/layers.js: projection dispatch by tensor name, shaped like
// matMulWeight / matMulWeightBatch / forwardOutput of
// packages/engine/src/runner/wasm/layers.ts.
import type { TopKCandidate } from "../hip-kernels";
import type { HipSession } from "./acceleration";

/* ForwardTrace (runtime.ts:70-73). */
export type HipTrace = {
  phase: string;
  onTiming(event: { phase: string; section: string; durationMs: number; weightName?: string }): void;
};

export function hipMatMulWeight(
  session: HipSession,
  weightName: string,
  inputColumns: Float32Array,
  trace?: HipTrace,
): Promise<Float32Array | undefined>;
export function hipMatMulWeightBatch(
  session: HipSession,
  weightNames: readonly string[],
  inputColumns: Float32Array,
  trace?: HipTrace,
): Promise<Float32Array[] | undefined>;
export function hipMatMulFfnGeglu(
  session: HipSession,
  gateName: string,
  upName: string,
  inputColumns: Float32Array,
  trace?: HipTrace,
): Promise<Float32Array | undefined>;
export function hipForwardOutputTopK(
  session: HipSession,
  normedHidden: Float32Array,
  topK: number,
  softcap?: number,
  trace?: HipTrace,
): Promise<TopKCandidate[][] | undefined>;
export function matMulWeight(
  session: HipSession,
  weightName: string,
  inputColumns: Float32Array,
  trace: HipTrace | undefined,
  fallback: (session: HipSession, weightName: string, inputColumns: Float32Array, trace?: HipTrace) => Promise<Float32Array>,
): Promise<Float32Array>;
export function matMulWeightBatch(
  session: HipSession,
  weightNames: readonly string[],
  inputColumns: Float32Array,
  trace: HipTrace | undefined,
  fallback?: (
    session: HipSession,
    weightNames: readonly string[],
    inputColumns: Float32Array,
    trace?: HipTrace,
  ) => Promise<Float32Array[] | undefined>,
): Promise<Float32Array[] | undefined>;
