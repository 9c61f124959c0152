"use strict";
/*
 * hip/layers.js -- projection dispatch by tensor name for the HIP runner.
 *
 * The decoder layers of packages/engine/src/runner/wasm/layers.ts reach every
 * weight through three calls; these are their HIP forms:
 *   matMulWeight 559-577 -> matMulKQ8K 751-797          matMulWeight / hipMatMulWeight
 *   matMulWeightBatch 585-716                           matMulWeightBatch / hipMatMulWeightBatch
 *   forwardFfn's gate/up batch + GeGLU 432-456          hipMatMulFfnGeglu
 *   forwardOutput's head + softcap + topK 381-416
 *     (runtime.ts topK 514-527)                         hipForwardOutputTopK
 *
 * The hip* functions answer undefined whenever the HIP runner cannot serve
 * the call (provider off, no GPU, a block type other than Q4_K/Q6_K, a
 * tensor whose shape the runner declines), exactly as the WASM resident
 * functions do, so the engine keeps its own path as the fallback; shape
 * mismatches of a call throw.  matMulWeight and matMulWeightBatch take that
 * fallback as their last argument (the engine passes its WASM
 * implementations) and call it when HIP answers undefined.
 *
 * Tensor shapes follow the engine: dimensions[0] is the input size and
 * dimensions[1] the row count (layers.ts:758-761); inputs are [columns][input]
 * f32 and outputs [columns][rows] f32.
 */

const acceleration = require("./acceleration.js");

const HIP_TYPES = new Set(["Q4_K", "Q6_K"]);

function tensorShape(session, name) {
  const tensor = session.getTensor(name);
  return {
    type: tensor.type,
    inputSize: (tensor.dimensions && tensor.dimensions[0]) || 0,
    rowCount: (tensor.dimensions && tensor.dimensions[1]) || 0,
  };
}

async function handleFor(session, name, shape) {
  if (!HIP_TYPES.has(shape.type) || shape.inputSize <= 0 || shape.rowCount <= 0) {
    return undefined;
  }
  return acceleration.readHipWeightHandle(session, name, shape.type, shape.inputSize, shape.rowCount);
}

function columnsOf(inputColumns, inputSize, name) {
  if (inputColumns.length % inputSize !== 0) {
    throw new Error(`${name} input shape mismatch: ${inputColumns.length} is not a multiple of ${inputSize}`);
  }
  return inputColumns.length / inputSize;
}

/* matMulKQ8K's resident step on the GPU: [columns][rows] f32, or undefined. */
async function hipMatMulWeight(session, weightName, inputColumns, trace) {
  if (!acceleration.hipExecutionProviderEnabled(session)) {
    return undefined;
  }
  const shape = tensorShape(session, weightName);
  const handle = await handleFor(session, weightName, shape);
  if (!handle) {
    return undefined;
  }
  const columnCount = columnsOf(inputColumns, shape.inputSize, weightName);
  return timed(trace, "HIP resident matmul", { weightName }, () =>
    acceleration.hipKernels().matMulQuantizedHipResident(handle, inputColumns, shape.inputSize, shape.rowCount,
                                                         columnCount));
}

/* matMulWeightBatch's resident step: 2..4 weights sharing the input, one
 * launch with one Q8_K quantisation per column; undefined when any weight
 * cannot run on the GPU (the engine then batches or loops on its own). */
async function hipMatMulWeightBatch(session, weightNames, inputColumns, trace) {
  if (!acceleration.hipProjectionBatchingEnabled(session) || weightNames.length < 2 || weightNames.length > 4) {
    return undefined;
  }
  const shapes = weightNames.map((name) => tensorShape(session, name));
  const inputSize = shapes[0].inputSize;
  if (inputSize <= 0 || shapes.some((shape) => shape.inputSize !== inputSize || !HIP_TYPES.has(shape.type))) {
    return undefined;
  }
  if (inputColumns.length % inputSize !== 0) {
    return undefined;
  }
  const handles = await Promise.all(weightNames.map((name, index) => handleFor(session, name, shapes[index])));
  if (!handles.every((handle) => handle !== undefined)) {
    return undefined;
  }
  const columnCount = inputColumns.length / inputSize;
  return timed(trace, "HIP resident matmul batch", {}, () =>
    acceleration.hipKernels().matMulQuantizedHipResidentMulti(handles, inputColumns, inputSize, columnCount));
}

/* forwardFfn's gate/up projections and GeGLU as one call: [columns][rows] of
 * fround(gelu(gate . x) * (up . x)), bit-exact with the engine's loop. */
async function hipMatMulFfnGeglu(session, gateName, upName, inputColumns, trace) {
  if (!acceleration.hipProjectionBatchingEnabled(session)) {
    return undefined;
  }
  const gateShape = tensorShape(session, gateName);
  const upShape = tensorShape(session, upName);
  if (gateShape.inputSize !== upShape.inputSize || gateShape.rowCount !== upShape.rowCount) {
    return undefined;
  }
  const [gate, up] = await Promise.all([handleFor(session, gateName, gateShape), handleFor(session, upName, upShape)]);
  if (!gate || !up) {
    return undefined;
  }
  const columnCount = columnsOf(inputColumns, gateShape.inputSize, gateName);
  return timed(trace, "HIP resident FFN gate/up + GeGLU", {}, () =>
    acceleration.hipKernels().matMulGegluHipResident(gate, up, inputColumns, gateShape.inputSize, columnCount));
}

/* forwardOutput after its final norm: the head's logits stay in HBM, the
 * softcap (manifest.finalLogitSoftcap, 0 = none) and topK run on the GPU,
 * and only the candidates come back: per column [{id, value}], best first.
 * The head is output.weight, else the tied token_embd.weight (layers.ts:397-399). */
async function hipForwardOutputTopK(session, normedHidden, topK, softcap, trace) {
  if (!acceleration.hipExecutionProviderEnabled(session)) {
    return undefined;
  }
  const tensors = session.tensorReader && session.tensorReader.metadata && session.tensorReader.metadata.tensors;
  const name = !tensors || tensors.some((tensor) => tensor.name === "output.weight") ? "output.weight"
    : "token_embd.weight";
  const shape = tensorShape(session, name);
  const handle = await handleFor(session, name, shape);
  if (!handle) {
    return undefined;
  }
  const columnCount = columnsOf(normedHidden, shape.inputSize, name);
  return timed(trace, "HIP output logits + topK", { weightName: name }, () =>
    acceleration.hipKernels().matMulQuantizedHipResidentTopK(handle, normedHidden, shape.inputSize, columnCount, topK,
                                                             softcap || 0));
}

/* matMulWeight with the HIP runner first and `fallback` (the engine's own
 * matMulWeight) when it answers undefined. */
async function matMulWeight(session, weightName, inputColumns, trace, fallback) {
  const hip = await hipMatMulWeight(session, weightName, inputColumns, trace);
  if (hip !== undefined) {
    return hip;
  }
  if (!fallback) {
    throw new Error(`HIP quantized matmul is unavailable for ${weightName} and no fallback was given.`);
  }
  return fallback(session, weightName, inputColumns, trace);
}

/* matMulWeightBatch with the HIP runner first; `fallback` (the engine's own
 * batch, which may itself answer undefined) otherwise. */
async function matMulWeightBatch(session, weightNames, inputColumns, trace, fallback) {
  const hip = await hipMatMulWeightBatch(session, weightNames, inputColumns, trace);
  if (hip !== undefined) {
    return hip;
  }
  return fallback ? fallback(session, weightNames, inputColumns, trace) : undefined;
}

/* The engine's timedAsync (runtime.ts:462-482): one timing event per call
 * on trace.onTiming, in the trace's phase. */
async function timed(trace, section, details, fn) {
  if (!trace || typeof trace.onTiming !== "function") {
    return fn();
  }
  const start = Date.now();
  try {
    return await fn();
  } finally {
    trace.onTiming(Object.assign({ phase: trace.phase, section, durationMs: Date.now() - start }, details));
  }
}

module.exports = {
  hipForwardOutputTopK,
  hipMatMulFfnGeglu,
  hipMatMulWeight,
  hipMatMulWeightBatch,
  matMulWeight,
  matMulWeightBatch,
};
