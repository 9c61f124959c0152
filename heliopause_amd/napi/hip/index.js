"use strict";
/*
 * hip/index.js -- the "hip" runner provider of packages/engine.
 *
 * Mirrors createWasmProvider / createWasmModelRunner
 * (packages/engine/src/runner/wasm/index.ts:45-87) and satisfies
 * ModelRunnerProvider (runner/provider.ts:30-36) with a ModelRunner
 * (runner/model-runner.ts:54-73) whose provider is "hip", the member this
 * runner adds to SegmentRunnerProvider (runner/segment-runner.ts:6).
 *
 * The HIP runner serves the quantized projections; the engine's WASM model
 * runner keeps the rest of the decoder (embedding, norms, RoPE, attention,
 * graph nodes), whose layers reach every weight through matMulWeight /
 * matMulWeightBatch / forwardOutput -- the calls hip/layers.js answers first.
 * The engine hands its pieces in as `engine`:
 *   engine.createWasmModelRunner            (wasm/index.ts:45-62)
 *   engine.createModelResourceRequirements  (runner/model-resources.ts:58-...)
 * so this module needs no engine import of its own.
 */

const acceleration = require("./acceleration.js");
const layers = require("./layers.js");
const segmentRunner = require("./segment-runner.js");

/* HBM of one MI355X: the whole model fits, so placement is full-model. */
const DEFAULT_HBM_BYTES = 288 * 1024 * 1024 * 1024;

function requireEngine(engine, member) {
  if (!engine || typeof engine[member] !== "function") {
    throw new Error(`The HIP runner provider needs engine.${member}.`);
  }
  return engine[member];
}

/* The engine's model runner with provider "hip".  A segment whose layers the
 * device path covers runs on HipSegmentRunner (hip/segment-runner.js: the
 * whole segment in HBM, one call per run); any other segment runs on the
 * engine's WASM segment runner, relabelled, whose projections go to
 * hip/layers.js. */
function createHipModelRunner(engine) {
  const base = requireEngine(engine, "createWasmModelRunner")();
  return Object.assign({}, base, {
    provider: "hip",
    segmentRunner: async (options) => {
      const device = await segmentRunner.createHipSegmentRunner(options);
      if (device) {
        return device;
      }
      const runner = await base.segmentRunner(options);
      return {
        provider: "hip",
        segmentStartLayer: runner.segmentStartLayer,
        segmentEndLayerExclusive: runner.segmentEndLayerExclusive,
        runTokensHidden: (...args) => runner.runTokensHidden(...args),
        runTokenHidden: (...args) => runner.runTokenHidden(...args),
      };
    },
  });
}

/* createHipProvider(options, engine): options are the provider's own
 * (residentWeightCache, projectionBatching: default true; memoryLimitBytes:
 * default one MI355X's HBM). */
function createHipProvider(options, engine) {
  const opts = Object.assign({}, options || {});
  return {
    name: "hip",
    options: opts,
    createModelRunner: () => createHipModelRunner(engine),
    modelResourceRequirements: (session, resourceOptions) =>
      requireEngine(engine, "createModelResourceRequirements")({
        provider: "hip",
        gguf: session.tensorReader.metadata,
        manifest: session.manifest,
        contextLength: resourceOptions.contextLength,
        slidingWindowReserveTokens: resourceOptions.slidingWindowReserveTokens,
        memoryLimitBytes: typeof opts.memoryLimitBytes === "number" ? opts.memoryLimitBytes : DEFAULT_HBM_BYTES,
        targetResourceConstrained: false,
        canRunFullModel: true,
        plannedReason: "HIP full-model placement is planned: every Q4_K/Q6_K weight resident in HBM.",
      }),
  };
}

module.exports = Object.assign({ DEFAULT_HBM_BYTES, createHipModelRunner, createHipProvider }, acceleration, layers,
  segmentRunner);
