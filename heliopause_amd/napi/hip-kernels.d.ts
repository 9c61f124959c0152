// Types of hip-kernels.js: the HIP runner's resident-weight API, shaped like
// packages/engine/src/runner/wasm/wasm-kernels.ts (WasmQuantizedWeightHandle
// 387-397, WasmResidentWeightStats 399-402, WasmSupport 404-408).

export type QuantizedType = "Q4_0" | "Q4_K" | "Q5_K" | "Q6_K" | "IQ4_XS" | "Q8_0";

export type HipQuantizedWeightHandle = {
  handle: bigint;
  type: QuantizedType;
  byteLength: number;
  rowCount: number;
  inputSize: number;
  released: boolean;
};

export type HipResidentWeightStats = {
  instanceCount: number;
  residentBytes: number;
  handleCount: number;
  scratchBytes: number;
  matmulCalls: number;
  kernelLaunches: number;
  device: number;
  computeUnits: number;
};

export type HipSupport = {
  available: boolean;
  reason?: "module-missing" | "device-missing";
  error?: string;
};

export type TopKCandidate = { id: number; value: number };

export function checkHipSupport(): Promise<HipSupport>;
export function quantizedTypeId(type: QuantizedType): number | undefined;
export function assertHipOk(code: number, kernelName: string, detail?: string): void;
export function createHipQuantizedWeightHandle(
  type: QuantizedType,
  weightBytes: Uint8Array,
  inputSize: number,
  rowCount: number,
): Promise<HipQuantizedWeightHandle | undefined>;
export function releaseHipQuantizedWeightHandle(handle: HipQuantizedWeightHandle): void;
export function hipResidentWeightStats(): HipResidentWeightStats;
export function matMulQuantizedHipResident(
  handle: HipQuantizedWeightHandle,
  inputColumns: Float32Array,
  inputSize: number,
  rowCount: number,
  columnCount: number,
): Promise<Float32Array>;
export function matMulQuantizedHipResidentMulti(
  handles: readonly HipQuantizedWeightHandle[],
  inputColumns: Float32Array,
  inputSize: number,
  columnCount: number,
): Promise<Float32Array[] | undefined>;
export function matMulQuantizedHipResidentTopK(
  handle: HipQuantizedWeightHandle,
  inputColumns: Float32Array,
  inputSize: number,
  columnCount: number,
  topK: number,
  softcap?: number,
): Promise<TopKCandidate[][]>;
export function matMulGegluHipResident(
  gate: HipQuantizedWeightHandle,
  up: HipQuantizedWeightHandle,
  inputColumns: Float32Array,
  inputSize: number,
  columnCount: number,
): Promise<Float32Array>;

// GGUF files (parseGguf's GgufMetadata shape, gguf.ts:30-37, plus byteLength).
export type HipGgufArraySummary = { type: string; length: number; sample: HipGgufMetadataValue[]; truncated: boolean };
export type HipGgufMetadataValue = number | boolean | string | HipGgufArraySummary;
export type HipGgufTensorInfo = {
  name: string;
  dimensions: number[];
  type: string;
  typeId: number;
  offset: bigint;
  dataOffset: bigint;
  byteLength?: number;
};
export type HipGgufMetadata = {
  version: number;
  tensorCount: number;
  metadataCount: number;
  metadata: Record<string, HipGgufMetadataValue>;
  tensors: HipGgufTensorInfo[];
  dataStart: bigint;
  alignment: number;
  fileSize: number;
};

export class HipGgufFile {
  constructor(path: string, options?: { maxArraySample?: number; completeArrayKeys?: readonly string[] });
  readonly metadata: HipGgufMetadata;
  getTensor(name: string): HipGgufTensorInfo;
  close(): void;
}
export function openHipGgufFile(
  path: string,
  options?: { maxArraySample?: number; completeArrayKeys?: readonly string[] },
): HipGgufFile;

export class HipGgufWeights {
  constructor(file: HipGgufFile);
  hits: number;
  misses: number;
  bytes: number;
  upload(names: readonly string[]): Promise<Map<string, HipQuantizedWeightHandle | undefined>>;
  handle(name: string): Promise<HipQuantizedWeightHandle | undefined>;
  release(): void;
}

// Token sampling on the device (generation.ts:40-165).
export const DEFAULT_SAMPLING_SEED: number;
export type ResolvedHipSamplingOptions = {
  doSample: boolean;
  temperature: number;
  topP: number;
  topK: number;
  seed: number;
  logitsTopK: number;
};
export function resolveGenerationSamplingOptions(options?: {
  doSample?: boolean;
  temperature?: number;
  topP?: number;
  topK?: number;
  seed?: number;
}): ResolvedHipSamplingOptions;
export function createHipSamplingState(seed?: number): Uint32Array;
export function matMulQuantizedHipResidentTopKSample(
  handle: HipQuantizedWeightHandle,
  inputColumns: Float32Array,
  inputSize: number,
  columnCount: number,
  sampling: ResolvedHipSamplingOptions,
  state: Uint32Array,
  softcap?: number,
): Promise<{ token: number; distribution: { id: number; value: number; probability: number }[] }[]>;

// Device buffers and the device-resident decode calls (hip/segment-runner.js).
export type HipDevicePointer = bigint;
export function deviceAlloc(bytes: number): HipDevicePointer;
export function deviceFree(ptr: HipDevicePointer): void;
export function copyToDevice(ptr: HipDevicePointer, array: ArrayBufferView, byteOffset?: number): void;
export function copyToHost(ptr: HipDevicePointer, array: ArrayBufferView, byteOffset?: number): void;
/* hp_hip_decode_layer_t as an object (include/hp_hip.h). */
export type HipDecodeLayerDescriptor = {
  attnQ: bigint; attnK: bigint; attnV: bigint; attnOutput: bigint; ffnGate: bigint; ffnUp: bigint; ffnDown: bigint;
  attnNorm: HipDevicePointer; attnQNorm: HipDevicePointer; attnKNorm: HipDevicePointer;
  postAttentionNorm: HipDevicePointer; ffnNorm: HipDevicePointer; postFfwNorm: HipDevicePointer;
  layerOutputScale: number;
  keyCache: HipDevicePointer; valueCache: HipDevicePointer;
  attention: {
    headCount: number; headCountKv: number; headDim: number; ropeDims: number; ropeFreqBase: number;
    ropeFreqFactors: HipDevicePointer; capacity: number; slidingWindow: number; epsilon: number;
  };
};
export function runDecodeLayers(
  layers: HipDecodeLayerDescriptor[],
  tokenCount: number,
  hiddenSize: number,
  buffers: { hidden: HipDevicePointer; position: HipDevicePointer; outputNorm: HipDevicePointer; output: HipDevicePointer },
  input: Float32Array | null,
  position: number,
  readOutput: boolean,
  rowStart: number,
  rowCount: number,
): Promise<Float32Array>;
export function headTopKDevice(
  handle: HipQuantizedWeightHandle,
  dInput: HipDevicePointer,
  inputSize: number,
  columnCount: number,
  topK: number,
  softcap?: number,
  sampling?: ResolvedHipSamplingOptions,
  state?: Uint32Array,
): Promise<unknown[]>;
