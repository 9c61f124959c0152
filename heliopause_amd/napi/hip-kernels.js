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

module.exports = {
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
