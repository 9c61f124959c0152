"use strict";
/*
 * hip-kernels.js -- the engine-side module of the HIP runner (CommonJS).
 *
 * Mirrors the resident-weight API of packages/engine/src/runner/wasm/
 * wasm-kernels.ts (same function shapes with Wasm -> Hip, same argument
 * meaning, same undefined-vs-throw behaviour) over the N-API addon
 * hp_hip.node, which calls the C ABI in include/hp_hip.h:
 *
 *   checkWasmSupport 1657-1675                 checkHipSupport
 *   createWasmQuantizedWeightHandle 520-574    createHipQuantizedWeightHandle
 *   releaseWasmQuantizedWeightHandle 576-584   releaseHipQuantizedWeightHandle
 *   wasmResidentWeightStats 586-591            hipResidentWeightStats
 *   matMulQuantizedWasmResident 593-646        matMulQuantizedHipResident
 *   matMulQuantizedWasmResidentMulti 648-749   matMulQuantizedHipResidentMulti
 *   assertWasmOk 1882-1896                     assertHipOk
 *   quantizedTypeId 1908-1923                  quantizedTypeId
 *   quantizedScaleValueCount 1925-1941         (its shape check, in create)
 *
 * the GGUF path that feeds them (file -> HBM without a JS copy):
 *   parseGguf (gguf.ts:150-215), GgufTensorReader.getTensor (tensor-reader.ts:66-72)
 *                                              openHipGgufFile -> HipGgufFile
 *   readWasmWeightHandle (acceleration.ts:164-201)
 *                                              HipGgufWeights.handle / upload
 *
 * token sampling on the device (generation.ts:40-165):
 *   resolveGenerationSamplingOptions           resolveGenerationSamplingOptions
 *   createDeterministicRng                     createHipSamplingState (state in a Uint32Array)
 *   forwardOutput + topK + sampleNextToken     matMulQuantizedHipResidentTopKSample
 *
 * plus the two calls the decode loop makes around the projections:
 *   forwardOutput + topK (layers.ts:381-416, runtime.ts:514-527)
 *                                              matMulQuantizedHipResidentTopK
 *   forwardFfn gate/up + GeGLU (layers.ts:432-456)
 *                                              matMulGegluHipResident
 *
 * Plain JavaScript (Node >= 12) so it runs without a TS build step; a .d.ts
 * beside it gives the types.  There is no CPU fallback here: when the addon
 * or the GPU is missing, checkHipSupport() says so and the calls throw.
 */

const path = require("path");

let addon;
let addonError;
try {
  addon = require(path.join(__dirname, "hp_hip.node"));
} catch (error) {
  addonError = error instanceof Error ? error.message : String(error);
}

const TYPE_IDS = { Q4_K: 1, Q5_K: 2, Q6_K: 3, IQ4_XS: 4, Q8_0: 5, Q4_0: 6 };
const HP_ERR_TYPE = 3;

function native() {
  if (!addon) {
    throw new Error(`HIP runner addon is not available: ${addonError}`);
  }
  return addon;
}

function quantizedTypeId(type) {
  return TYPE_IDS[type];
}

function assertHipOk(code, kernelName, detail) {
  if (code === 0) {
    return;
  }
  if (code === 1) {
    throw new Error(`${kernelName} hip shape mismatch`);
  }
  if (code === 2) {
    throw new Error(`${kernelName} hip head count mismatch`);
  }
  if (code === 3) {
    throw new Error(`${kernelName} hip unsupported type`);
  }
  const message = detail !== undefined ? detail : addon ? addon.lastError() : "";
  throw new Error(`${kernelName} hip failed with code ${code} (${message})`);
}

async function checkHipSupport() {
  if (!addon) {
    return { available: false, reason: "module-missing", error: addonError };
  }
  if (addon.deviceCount() <= 0) {
    return { available: false, reason: "device-missing" };
  }
  return { available: true };
}

async function createHipQuantizedWeightHandle(type, weightBytes, inputSize, rowCount) {
  const typeId = quantizedTypeId(type);
  if (!typeId) {
    return undefined;
  }
  if (inputSize <= 0 || rowCount <= 0) {
    throw new Error(`Resident quantized weight shape mismatch: inputSize=${inputSize} rowCount=${rowCount}`);
  }
  const blockValues = type === "Q4_0" || type === "Q8_0" ? 32 : 256;
  if (inputSize % blockValues !== 0) {
    throw new Error(`${type} scale shape mismatch: ${inputSize}`);
  }
  const result = native().upload(typeId, weightBytes, inputSize, rowCount);
  if (result.status === HP_ERR_TYPE) {
    return undefined; // a type this runner does not implement: the caller falls back
  }
  assertHipOk(result.status, "createQuantizedWeightHandle");
  return {
    handle: result.handle,
    type,
    byteLength: weightBytes.byteLength,
    rowCount,
    inputSize,
    released: false,
  };
}

function releaseHipQuantizedWeightHandle(handle) {
  if (!addon || !handle || handle.released) {
    return;
  }
  addon.release(handle.handle);
  handle.released = true;
}

function hipResidentWeightStats() {
  const s = native().stats();
  assertHipOk(s.status, "residentWeightStats");
  return {
    instanceCount: s.device >= 0 ? 1 : 0,
    residentBytes: s.residentBytes,
    handleCount: s.handleCount,
    scratchBytes: s.scratchBytes,
    matmulCalls: s.matmulCalls,
    kernelLaunches: s.kernelLaunches,
    device: s.device,
    computeUnits: s.computeUnits,
  };
}

async function matMulQuantizedHipResident(handle, inputColumns, inputSize, rowCount, columnCount) {
  if (handle.released) {
    throw new Error(`Resident quantized matmul instance ${handle.handle} is not available`);
  }
  if (handle.inputSize !== inputSize || handle.rowCount !== rowCount) {
    throw new Error(`Resident quantized matmul handle shape mismatch: ${handle.inputSize}x${handle.rowCount}`);
  }
  if (inputColumns.length !== inputSize * columnCount) {
    throw new Error(`Resident quantized matmul input shape mismatch: ${inputColumns.length}`);
  }
  if (!quantizedTypeId(handle.type)) {
    throw new Error(`Resident quantized matmul type ${handle.type} is not supported`);
  }
  const result = await native().matmulMulti([handle.handle], inputColumns, inputSize, columnCount, [rowCount]);
  assertHipOk(result.status, "matMulQuantizedResident", result.error);
  return result.outputs[0];
}

async function matMulQuantizedHipResidentMulti(handles, inputColumns, inputSize, columnCount) {
  if (handles.length < 2 || handles.length > 4) {
    return undefined;
  }
  if (inputColumns.length !== inputSize * columnCount) {
    throw new Error(`Resident quantized multi matmul input shape mismatch: ${inputColumns.length}`);
  }
  for (const handle of handles) {
    if (handle.inputSize !== inputSize) {
      throw new Error(`Resident quantized multi matmul handle shape mismatch: ${handle.inputSize}`);
    }
    if (handle.released) {
      throw new Error(`Resident quantized multi matmul instance ${handle.handle} is not available`);
    }
  }
  if (handles.some((handle) => !quantizedTypeId(handle.type))) {
    throw new Error("Resident quantized multi matmul has unsupported type");
  }
  const result = await native().matmulMulti(
    handles.map((handle) => handle.handle),
    inputColumns,
    inputSize,
    columnCount,
    handles.map((handle) => handle.rowCount),
  );
  assertHipOk(result.status, "MatMulQuantizedResidentMulti", result.error);
  return result.outputs;
}

/* Output head + topK per column: the logits stay in HBM and only the
 * candidates come back, [{id, value}] per column, best first. */
async function matMulQuantizedHipResidentTopK(handle, inputColumns, inputSize, columnCount, topK, softcap) {
  if (handle.released) {
    throw new Error(`Resident quantized matmul instance ${handle.handle} is not available`);
  }
  if (handle.inputSize !== inputSize || inputColumns.length !== inputSize * columnCount) {
    throw new Error(`Resident quantized matmul input shape mismatch: ${inputColumns.length}`);
  }
  const result = await native().matmulTopK(
    handle.handle,
    inputColumns,
    inputSize,
    columnCount,
    topK,
    softcap === undefined ? 0 : softcap,
  );
  assertHipOk(result.status, "matMulQuantizedResidentTopK", result.error);
  const count = Math.min(handle.rowCount, topK);
  const columns = [];
  for (let column = 0; column < columnCount; column += 1) {
    const candidates = [];
    for (let index = 0; index < count; index += 1) {
      candidates.push({ id: result.ids[column * topK + index], value: result.values[column * topK + index] });
    }
    columns.push(candidates);
  }
  return columns;
}

/* forwardFfn's gate/up batch and GeGLU: [columnCount][rowCount] of
 * fround(gelu(gate . x) * (up . x)). */
async function matMulGegluHipResident(gate, up, inputColumns, inputSize, columnCount) {
  for (const handle of [gate, up]) {
    if (handle.released) {
      throw new Error(`Resident quantized matmul instance ${handle.handle} is not available`);
    }
  }
  if (gate.inputSize !== inputSize || up.inputSize !== inputSize || inputColumns.length !== inputSize * columnCount) {
    throw new Error(`Resident quantized matmul input shape mismatch: ${inputColumns.length}`);
  }
  if (gate.rowCount !== up.rowCount) {
    throw new Error(`Resident quantized matmul handle shape mismatch: ${gate.rowCount}x${up.rowCount}`);
  }
  const result = await native().matmulGeglu(
    gate.handle,
    up.handle,
    inputColumns,
    inputSize,
    columnCount,
    gate.rowCount,
  );
  assertHipOk(result.status, "matMulGegluResident", result.error);
  return result.output;
}

const DEFAULT_SAMPLING_SEED = 0x48454c49;

/* resolveGenerationSamplingOptions (generation.ts:40-76). */
function resolveGenerationSamplingOptions(options) {
  const o = options || {};
  const doSample = o.doSample === undefined ? true : o.doSample;
  const temperature = o.temperature === undefined ? 1.0 : o.temperature;
  const topP = o.topP === undefined ? 0.95 : o.topP;
  const topK = o.topK === undefined ? 64 : o.topK;
  const seed = o.seed === undefined ? DEFAULT_SAMPLING_SEED : o.seed;
  if (!Number.isFinite(temperature) || temperature < 0) {
    throw new Error("temperature must be a finite number greater than or equal to 0.");
  }
  if (!Number.isFinite(topP) || topP <= 0 || topP > 1) {
    throw new Error("topP must be a finite number in the range (0, 1].");
  }
  if (!Number.isFinite(topK) || topK < 1) {
    throw new Error("topK must be a positive finite number.");
  }
  if (!Number.isFinite(seed)) {
    throw new Error("seed must be a finite number.");
  }
  const normalizedTopK = Math.max(1, Math.floor(topK));
  const greedy = doSample === false || temperature === 0;
  return {
    doSample,
    temperature,
    topP,
    topK: normalizedTopK,
    seed: Math.floor(seed) >>> 0,
    logitsTopK: greedy ? 1 : normalizedTopK,
  };
}

/* The generator of createDeterministicRng (generation.ts:78-87) as the
 * 32-bit state the GPU advances, one draw per sampled column. */
function createHipSamplingState(seed) {
  return Uint32Array.of(Math.floor(seed === undefined ? DEFAULT_SAMPLING_SEED : seed) >>> 0);
}

/* forwardOutput + topK + sampleNextToken per column on the GPU; `sampling`
 * is resolved options, `state` a createHipSamplingState array (advanced).
 * Returns [{token, distribution: [{id, value, probability}]}] per column. */
async function matMulQuantizedHipResidentTopKSample(handle, inputColumns, inputSize, columnCount, sampling, state,
  softcap) {
  if (handle.released) {
    throw new Error(`Resident quantized matmul instance ${handle.handle} is not available`);
  }
  if (handle.inputSize !== inputSize || inputColumns.length !== inputSize * columnCount) {
    throw new Error(`Resident quantized matmul input shape mismatch: ${inputColumns.length}`);
  }
  const k = sampling.logitsTopK;
  const result = await native().matmulTopKSample(handle.handle, inputColumns, inputSize, columnCount, k,
    softcap === undefined ? 0 : softcap, sampling, state);
  assertHipOk(result.status, "matMulQuantizedResidentTopKSample", result.error);
  const columns = [];
  for (let column = 0; column < columnCount; column += 1) {
    const distribution = [];
    for (let index = 0; index < result.kept[column]; index += 1) {
      const at = column * k + index;
      distribution.push({ id: result.ids[at], value: result.values[at], probability: result.probabilities[at] });
    }
    columns.push({ token: result.tokens[column], distribution });
  }
  return columns;
}

/* Device buffers and the device-resident decode calls behind the segment
 * runner (hip/segment-runner.js): BigInt device addresses of
 * hp_hip_device_alloc, copies that return once the bytes have arrived, and
 * the layer / head calls on device rows (hp_hip.h). */
function deviceAlloc(bytes) {
  const result = native().deviceAlloc(bytes);
  assertHipOk(result.status, "deviceAlloc");
  return result.ptr;
}

function deviceFree(ptr) {
  if (addon && ptr) {
    assertHipOk(addon.deviceFree(ptr), "deviceFree");
  }
}

function copyToDevice(ptr, array, byteOffset) {
  assertHipOk(native().copyToDevice(ptr, array, byteOffset || 0), "copyToDevice");
}

function copyToHost(ptr, array, byteOffset) {
  assertHipOk(native().copyToHost(ptr, array, byteOffset || 0), "copyToHost");
}

/* hp_hip_decode_layers_device over `layers` (runLayers objects) for
 * tokenCount tokens at `position` ..: `input` rows (or null: already in
 * buffers.hidden), then rows [rowStart, rowStart + rowCount) of the residual
 * stream (readOutput false) or of the output norm read back. */
async function runDecodeLayers(layers, tokenCount, hiddenSize, buffers, input, position, readOutput, rowStart,
  rowCount) {
  const result = await native().runLayers(layers, tokenCount, hiddenSize, buffers, input, position, readOutput,
    rowStart, rowCount);
  assertHipOk(result.status, "decodeLayers", result.error);
  return result.output;
}

/* forwardOutput's head + topK (+ sampleNextToken with `sampling` and a
 * createHipSamplingState `state`) on device rows: [{id, value}] per column,
 * or with sampling [{token, distribution}] as matMulQuantizedHipResidentTopKSample. */
async function headTopKDevice(handle, dInput, inputSize, columnCount, topK, softcap, sampling, state) {
  if (handle.released) {
    throw new Error(`Resident quantized matmul instance ${handle.handle} is not available`);
  }
  if (handle.inputSize !== inputSize) {
    throw new Error(`Resident quantized matmul input shape mismatch: ${inputSize}`);
  }
  const k = sampling ? sampling.logitsTopK : topK;
  const result = await native().headTopK(handle.handle, dInput, inputSize, columnCount, k,
    softcap === undefined ? 0 : softcap, sampling || null, sampling ? state : null);
  assertHipOk(result.status, "headTopK", result.error);
  const columns = [];
  for (let column = 0; column < columnCount; column += 1) {
    if (sampling) {
      const distribution = [];
      for (let index = 0; index < result.kept[column]; index += 1) {
        const at = column * k + index;
        distribution.push({ id: result.ids[at], value: result.values[at], probability: result.probabilities[at] });
      }
      columns.push({ token: result.tokens[column], distribution });
    } else {
      const candidates = [];
      for (let index = 0; index < Math.min(handle.rowCount, k); index += 1) {
        candidates.push({ id: result.ids[column * k + index], value: result.values[column * k + index] });
      }
      columns.push(candidates);
    }
  }
  return columns;
}

/* A GGUF file parsed by the runner's reader and held open for uploads.
 * `metadata` has parseGguf's shape (GgufMetadata, gguf.ts:30-37), with each
 * tensor's byteLength (tensorByteLength) when its storage type is known. */
class HipGgufFile {
  constructor(path, options) {
    const opts = options || {};
    const result = native().ggufOpen(
      path,
      opts.maxArraySample === undefined ? 16 : opts.maxArraySample,
      opts.completeArrayKeys || [],
    );
    if (result.status !== 0) {
      throw new Error(result.error);
    }
    this.file = result.file;
    this.metadata = native().ggufInfo(this.file);
    this.tensorsByName = new Map(this.metadata.tensors.map((tensor, index) => [tensor.name, index]));
  }

  getTensor(name) {
    const index = this.tensorsByName.get(name);
    if (index === undefined) {
      throw new Error(`Unknown tensor: ${name}`);
    }
    return this.metadata.tensors[index];
  }

  close() {
    if (this.file) {
      native().ggufClose(this.file);
      this.file = undefined;
    }
  }
}

function openHipGgufFile(path, options) {
  return new HipGgufFile(path, options);
}

/* Session cache of HBM-resident handles keyed by tensor name
 * (readWasmWeightHandle, acceleration.ts:164-201): a hit returns the cached
 * handle, a pending upload is shared, a miss uploads.  upload(names) loads
 * many tensors in one streamed call.  Block types the runner does not
 * implement resolve to undefined, so the engine falls back. */
class HipGgufWeights {
  constructor(file) {
    this.file = file;
    this.handles = new Map();
    this.pending = new Map();
    this.unsupported = new Set();
    this.hits = 0;
    this.misses = 0;
    this.bytes = 0;
  }

  async upload(names) {
    const todo = [];
    for (const name of new Set(names)) {
      if (!this.handles.has(name) && !this.pending.has(name) && !this.unsupported.has(name)) {
        todo.push(name);
      }
    }
    if (todo.length > 0) {
      const tensors = todo.map((name) => this.file.getTensor(name));
      const run = native()
        .ggufUpload(this.file.file, todo.map((name) => this.file.tensorsByName.get(name)))
        .then((result) => {
          assertHipOk(result.status, "uploadGgufWeights", result.error);
          tensors.forEach((tensor, index) => {
            if (result.statuses[index] !== 0) {
              this.unsupported.add(tensor.name);
              return;
            }
            this.handles.set(tensor.name, {
              handle: result.handles[index],
              type: tensor.type,
              byteLength: tensor.byteLength,
              rowCount: tensor.dimensions[1],
              inputSize: tensor.dimensions[0],
              released: false,
            });
            this.bytes += tensor.byteLength;
          });
        });
      const settled = run.then(() => undefined, () => undefined);
      for (const name of todo) {
        this.pending.set(name, settled);
      }
      try {
        await run;
      } finally {
        for (const name of todo) {
          this.pending.delete(name);
        }
      }
    }
    await Promise.all(names.map((name) => this.pending.get(name)).filter((p) => p !== undefined));
    const out = new Map();
    for (const name of names) {
      out.set(name, this.handles.get(name));
    }
    return out;
  }

  async handle(name) {
    if (this.handles.has(name) || this.unsupported.has(name)) {
      this.hits += 1;
      return this.handles.get(name);
    }
    if (this.pending.has(name)) {
      this.hits += 1;
      await this.pending.get(name);
      return this.handles.get(name);
    }
    this.misses += 1;
    return (await this.upload([name])).get(name);
  }

  release() {
    for (const handle of this.handles.values()) {
      releaseHipQuantizedWeightHandle(handle);
    }
    this.handles.clear();
    this.bytes = 0;
  }
}

module.exports = {
  DEFAULT_SAMPLING_SEED,
  copyToDevice,
  copyToHost,
  deviceAlloc,
  deviceFree,
  headTopKDevice,
  runDecodeLayers,
  createHipSamplingState,
  matMulQuantizedHipResidentTopKSample,
  resolveGenerationSamplingOptions,
  HipGgufFile,
  HipGgufWeights,
  openHipGgufFile,
  assertHipOk,
  checkHipSupport,
  createHipQuantizedWeightHandle,
  hipResidentWeightStats,
  matMulGegluHipResident,
  matMulQuantizedHipResident,
  matMulQuantizedHipResidentMulti,
  matMulQuantizedHipResidentTopK,
  quantizedTypeId,
  releaseHipQuantizedWeightHandle,
};
