"use strict";
// Drives the engine-side HIP runner (heliopause_amd/napi/hip/) from Node.
//   node hip_runner_driver.js dispatch   -> JSON of the dispatch checks with a stand-in
//                                           runner module and a mock session (no GPU)
//   node hip_runner_driver.js nogpu      -> JSON: the real runner module on a host
//                                           without a GPU answers undefined, the fallback runs
//   node hip_runner_driver.js layer <dir> -> one decoder layer's projections by tensor name
//                                           over <dir>/model.gguf (GPU); writes out_*.bin
const fs = require("fs");
const path = require("path");

const HIP = path.join(__dirname, "..", "heliopause_amd", "napi", "hip", "index.js");

async function throws(fn) {
  try {
    await fn();
    return "";
  } catch (error) {
    return error.message;
  }
}

/* A ModelSession stand-in: tensors from a table, providers from a list. */
function mockSession(tensors, providers, hipOptions) {
  const statsProviders = {};
  return {
    statsProviders,
    reads: [],
    hasProvider: (name) => providers.includes(name),
    provider: (name) => (name === "hip" && providers.includes("hip") ? { name: "hip", options: hipOptions || {} } : undefined),
    setExecutionProviderStatsProvider(fn, name) {
      statsProviders[name] = fn;
    },
    getTensor(name) {
      const t = tensors[name];
      if (!t) {
        throw new Error(`Unknown tensor: ${name}`);
      }
      return t;
    },
    tensorReader: {
      metadata: { tensors: Object.keys(tensors).map((name) => ({ name })) },
      async readTensorBytes(name) {
        this.owner.reads.push(name);
        return new Uint8Array(tensors[name].bytes || 16);
      },
    },
  };
}

/* Runner module stand-in: records calls; a handle's rowCount answers the
 * matmul with row-index values so outputs are checkable. */
function fakeKernels(log) {
  let next = 1;
  return {
    checkHipSupport: async () => ({ available: true }),
    quantizedTypeId: (t) => ({ Q4_K: 1, Q5_K: 2, Q6_K: 3, IQ4_XS: 4, Q8_0: 5, Q4_0: 6 })[t],
    async createHipQuantizedWeightHandle(type, bytes, inputSize, rowCount) {
      log.push(`create ${type} ${inputSize}x${rowCount}`);
      if (type === "Q5_K") {
        return undefined; // the runner declines this type
      }
      if (rowCount === 13) {
        throw new Error("Resident quantized weight shape mismatch: inputSize=256 rowCount=13");
      }
      await new Promise((resolve) => setTimeout(resolve, 5));
      return { handle: BigInt(next++), type, byteLength: bytes.byteLength, rowCount, inputSize, released: false };
    },
    releaseHipQuantizedWeightHandle(h) {
      log.push(`release ${h.handle}`);
      h.released = true;
    },
    async matMulQuantizedHipResident(h, x, inputSize, rowCount, columns) {
      log.push(`matmul ${h.handle}`);
      return Float32Array.from({ length: rowCount * columns }, (_, i) => i % rowCount);
    },
    async matMulQuantizedHipResidentMulti(hs, x, inputSize, columns) {
      log.push(`multi ${hs.map((h) => h.handle).join(",")}`);
      return hs.map((h) => new Float32Array(h.rowCount * columns).fill(Number(h.handle)));
    },
    async matMulGegluHipResident(g, u, x, inputSize, columns) {
      log.push(`geglu ${g.handle},${u.handle}`);
      return new Float32Array(g.rowCount * columns).fill(7);
    },
    async matMulQuantizedHipResidentTopK(h, x, inputSize, columns, topK, softcap) {
      log.push(`topk ${h.handle} k=${topK} softcap=${softcap}`);
      return Array.from({ length: columns }, () => [{ id: 3, value: 1.5 }]);
    },
  };
}

async function dispatch() {
  const hip = require(HIP);
  const log = [];
  hip.setHipKernels(fakeKernels(log));
  const tensors = {
    "blk.0.attn_q.weight": { type: "Q4_K", dimensions: [256, 8] },
    "blk.0.attn_k.weight": { type: "Q4_K", dimensions: [256, 4] },
    "blk.0.attn_v.weight": { type: "Q6_K", dimensions: [256, 4] },
    "blk.0.attn_norm.weight": { type: "F32", dimensions: [256] },
    "blk.0.ffn_gate.weight": { type: "Q4_K", dimensions: [256, 6] },
    "blk.0.ffn_up.weight": { type: "Q4_K", dimensions: [256, 6] },
    "blk.0.odd.weight": { type: "Q5_K", dimensions: [256, 4] },
    "blk.0.q8.weight": { type: "Q8_0", dimensions: [256, 4] },
    "blk.0.bad.weight": { type: "Q4_K", dimensions: [256, 13] },
    "output.weight": { type: "Q6_K", dimensions: [256, 100] },
  };
  const session = mockSession(tensors, ["wasm", "hip"]);
  session.tensorReader.owner = session;
  const fallbackCalls = [];
  const fallback = async (s, name, x) => {
    fallbackCalls.push(name);
    return new Float32Array(2).fill(-1);
  };
  const batchFallback = async (s, names) => {
    fallbackCalls.push(names.join("+"));
    return undefined;
  };
  const x = new Float32Array(512); // two columns of 256
  hip.registerHipExecutionProvider(session);
  const out = {};
  // one weight: the HIP handle serves it; repeated and concurrent calls share the upload
  const [a, b] = await Promise.all([
    hip.matMulWeight(session, "blk.0.attn_q.weight", x, undefined, fallback),
    hip.matMulWeight(session, "blk.0.attn_q.weight", x, undefined, fallback),
  ]);
  out.single = Array.from(a.slice(0, 10));
  out.singleConcurrentSame = Array.from(b).join() === Array.from(a).join();
  out.reads = session.reads.slice();
  // a batch of Q/K/V: one multi call
  out.batch = (await hip.matMulWeightBatch(session, ["blk.0.attn_q.weight", "blk.0.attn_k.weight",
    "blk.0.attn_v.weight"], x, undefined, batchFallback)).map((o) => o.length);
  // a batch with a type the runner declines: the engine's batch runs instead
  out.batchDeclined = String(await hip.matMulWeightBatch(session, ["blk.0.attn_q.weight", "blk.0.odd.weight"], x,
    undefined, batchFallback));
  // a type HIP never takes (Q8_0) and a dense F32 tensor: fallback
  out.q8 = Array.from(await hip.matMulWeight(session, "blk.0.q8.weight", x, undefined, fallback));
  out.f32 = Array.from(await hip.matMulWeight(session, "blk.0.attn_norm.weight", x, undefined, fallback));
  // a declined type is asked once, then remembered
  out.odd1 = String(await hip.hipMatMulWeight(session, "blk.0.odd.weight", x));
  out.odd2 = String(await hip.hipMatMulWeight(session, "blk.0.odd.weight", x));
  // shape errors throw (no fallback)
  out.badHandle = await throws(() => hip.matMulWeight(session, "blk.0.bad.weight", x, undefined, fallback));
  out.badInput = await throws(() => hip.matMulWeight(session, "blk.0.attn_q.weight", new Float32Array(300), undefined,
    fallback));
  out.noFallback = await throws(() => hip.matMulWeight(session, "blk.0.q8.weight", x));
  // batch sizes outside 2..4 are not batched
  out.batchOne = String(await hip.hipMatMulWeightBatch(session, ["blk.0.attn_q.weight"], x));
  // FFN gate/up + GeGLU and the head's top-k
  out.geglu = (await hip.hipMatMulFfnGeglu(session, "blk.0.ffn_gate.weight", "blk.0.ffn_up.weight", x)).length;
  out.topk = await hip.hipForwardOutputTopK(session, x, 40, 30);
  out.fallbackCalls = fallbackCalls;
  out.stats = session.statsProviders.hip();
  // provider switched off, and options that turn the cache or batching off
  const off = mockSession(tensors, ["wasm"]);
  off.tensorReader.owner = off;
  out.offSingle = String(await hip.hipMatMulWeight(off, "blk.0.attn_q.weight", x));
  out.offFallback = Array.from(await hip.matMulWeight(off, "blk.0.attn_q.weight", x, undefined, fallback));
  const noCache = mockSession(tensors, ["hip"], { residentWeightCache: false });
  noCache.tensorReader.owner = noCache;
  out.noCache = String(await hip.hipMatMulWeight(noCache, "blk.0.attn_q.weight", x));
  const noBatch = mockSession(tensors, ["hip"], { projectionBatching: false });
  noBatch.tensorReader.owner = noBatch;
  out.noBatch = String(await hip.hipMatMulWeightBatch(noBatch, ["blk.0.attn_q.weight", "blk.0.attn_k.weight"], x));
  // shutdown releases every handle of the session
  hip.shutdownHipExecutionProvider(session);
  out.afterShutdown = session.statsProviders.hip();
  out.log = log;
  // the provider object
  const engine = {
    createWasmModelRunner: () => ({
      provider: "wasm",
      graphNodes: { marker: 1 },
      prepareInput: async () => "prepared",
      segmentRunner: async (options) => ({
        provider: "wasm",
        segmentStartLayer: options.segmentStartLayer,
        segmentEndLayerExclusive: options.segmentEndLayerExclusive,
        runTokensHidden: async () => ({ hidden: new Float32Array(1) }),
        runTokenHidden: async () => ({ hidden: new Float32Array(2) }),
      }),
    }),
    createModelResourceRequirements: (o) => o,
  };
  const provider = hip.createHipProvider({ projectionBatching: true }, engine);
  const runner = provider.createModelRunner();
  const seg = await runner.segmentRunner({ segmentStartLayer: 2, segmentEndLayerExclusive: 5 });
  out.provider = {
    name: provider.name,
    options: provider.options,
    runnerProvider: runner.provider,
    graphNodes: runner.graphNodes,
    prepared: await runner.prepareInput(),
    segment: [seg.provider, seg.segmentStartLayer, seg.segmentEndLayerExclusive],
    tokensHidden: (await seg.runTokensHidden()).hidden.length,
    tokenHidden: (await seg.runTokenHidden()).hidden.length,
    requirements: provider.modelResourceRequirements(
      { tensorReader: { metadata: "gguf" }, manifest: "manifest" }, { contextLength: 4096 }),
  };
  out.missingEngine = await throws(() => hip.createHipProvider({}, {}).createModelRunner());
  process.stdout.write(JSON.stringify(out));
}

async function nogpu() {
  const hip = require(HIP);
  const tensors = { "blk.0.attn_q.weight": { type: "Q4_K", dimensions: [256, 8] } };
  const session = mockSession(tensors, ["wasm", "hip"]);
  session.tensorReader.owner = session;
  const support = await hip.hipKernels().checkHipSupport();
  const called = [];
  const out = await hip.matMulWeight(session, "blk.0.attn_q.weight", new Float32Array(256), undefined,
    async (s, name) => {
      called.push(name);
      return new Float32Array([1, 2]);
    });
  process.stdout.write(JSON.stringify({ support, out: Array.from(out), called, stats: hip.hipExecutionProviderStats(session) }));
}

function readF32(file) {
  const b = fs.readFileSync(file);
  return new Float32Array(b.buffer, b.byteOffset, b.byteLength / 4);
}

function writeF32(file, a) {
  fs.writeFileSync(file, Buffer.from(a.buffer, a.byteOffset, a.byteLength));
}

/* A session over a GGUF file: tensors from the runner's GGUF reader, bytes
 * read from the file range (the engine's tensorReader.readTensorBytes). */
function fileSession(file) {
  const kernels = require(path.join(__dirname, "..", "heliopause_amd", "napi", "hip-kernels.js"));
  const gguf = kernels.openHipGgufFile(file);
  const fd = fs.openSync(file, "r");
  const session = mockSession({}, ["wasm", "hip"]);
  session.getTensor = (name) => gguf.getTensor(name);
  session.tensorReader = {
    metadata: gguf.metadata,
    async readTensorBytes(name) {
      const t = gguf.getTensor(name);
      const out = Buffer.alloc(t.byteLength);
      fs.readSync(fd, out, 0, t.byteLength, Number(t.dataOffset));
      session.reads.push(name);
      return new Uint8Array(out.buffer, out.byteOffset, out.byteLength);
    },
  };
  session.close = () => {
    fs.closeSync(fd);
    gguf.close();
  };
  return session;
}

async function layer(dir) {
  const hip = require(HIP);
  const spec = JSON.parse(fs.readFileSync(path.join(dir, "case.json"), "utf8"));
  const session = fileSession(path.join(dir, "model.gguf"));
  hip.registerHipExecutionProvider(session);
  const x = (name) => readF32(path.join(dir, `${name}.bin`));
  const fallbackCalls = [];
  const fallback = async (s, name) => {
    fallbackCalls.push(name);
    return new Float32Array(1);
  };
  const qkv = await hip.matMulWeightBatch(session, ["blk.0.attn_q.weight", "blk.0.attn_k.weight",
    "blk.0.attn_v.weight"], x("x_attn"), undefined, async () => undefined);
  qkv.forEach((o, i) => writeF32(path.join(dir, `out_qkv${i}.bin`), o));
  writeF32(path.join(dir, "out_o.bin"), await hip.matMulWeight(session, "blk.0.attn_output.weight", x("x_o"),
    undefined, fallback));
  writeF32(path.join(dir, "out_ffn.bin"), await hip.hipMatMulFfnGeglu(session, "blk.0.ffn_gate.weight",
    "blk.0.ffn_up.weight", x("x_ffn")));
  const gateUp = await hip.matMulWeightBatch(session, ["blk.0.ffn_gate.weight", "blk.0.ffn_up.weight"], x("x_ffn"),
    undefined, async () => undefined);
  gateUp.forEach((o, i) => writeF32(path.join(dir, `out_gateup${i}.bin`), o));
  writeF32(path.join(dir, "out_down.bin"), await hip.matMulWeight(session, "blk.0.ffn_down.weight", x("x_down"),
    undefined, fallback));
  const top = await hip.hipForwardOutputTopK(session, x("x_head"), spec.topK, spec.softcap);
  // a dense tensor goes to the engine's path
  await hip.matMulWeight(session, "blk.0.attn_norm.weight", x("x_attn"), undefined, fallback);
  const stats = session.statsProviders.hip();
  hip.shutdownHipExecutionProvider(session);
  session.close();
  process.stdout.write(JSON.stringify({ top, fallbackCalls, stats, reads: session.reads }));
}

/* A device stand-in over fakeKernels: buffers are host byte arrays behind
 * BigInt addresses; the layer call records its arguments and answers rows
 * whose values name the row and the position. */
function fakeDevice(log) {
  const k = fakeKernels(log);
  let nextPtr = 0x10000n;
  const buffers = new Map();
  const calls = [];
  return Object.assign(k, {
    buffers,
    calls,
    deviceAlloc(bytes) {
      const ptr = nextPtr;
      nextPtr += BigInt(bytes + 4096);
      buffers.set(ptr, new Uint8Array(bytes));
      log.push(`alloc ${bytes}`);
      return ptr;
    },
    deviceFree(ptr) {
      if (!buffers.delete(ptr)) {
        throw new Error(`free of an unknown buffer ${ptr}`);
      }
      log.push("free");
    },
    copyToDevice(ptr, array, byteOffset) {
      buffers.get(ptr).set(new Uint8Array(array.buffer, array.byteOffset, array.byteLength), byteOffset || 0);
    },
    copyToHost(ptr, array, byteOffset) {
      const b = buffers.get(ptr);
      new Uint8Array(array.buffer, array.byteOffset, array.byteLength).set(
        b.subarray(byteOffset || 0, (byteOffset || 0) + array.byteLength));
    },
    async runDecodeLayers(layers, tokenCount, hiddenSize, bufs, input, position, readOutput, rowStart, rowCount) {
      calls.push({ layers, tokenCount, hiddenSize, bufs, inputLength: input ? input.length : -1, position, readOutput,
        rowStart, rowCount });
      return Float32Array.from({ length: rowCount * hiddenSize },
        (_, i) => (rowStart + Math.floor(i / hiddenSize)) * 1000 + position);
    },
    async headTopKDevice(handle, dInput, inputSize, columns, topK, softcap, sampling) {
      calls.push({ head: String(handle.handle), dInput: String(dInput), inputSize, columns, topK, softcap,
        sampling: Boolean(sampling) });
      return [[{ id: 7, value: 2.5 }, { id: 3, value: 1.5 }]];
    },
  });
}

/* A Gemma-like manifest of `layers` layers (even: sliding, odd: full). */
function manifestOf(layers, extra) {
  const m = {
    blockCount: layers, embeddingLength: 512, headCount: 4, headCountKv: 2, layerHeadCountKv: [],
    keyLength: 256, valueLength: 256, layerKeyLengths: [], layerValueLengths: [],
    layerHasKv: Array(layers).fill(true), layerValueProjectionModes: Array(layers).fill("separate"),
    kvSourceLayers: [], slidingWindow: 48, perLayerEmbeddingLength: 0,
    layerKinds: Array.from({ length: layers }, (_, i) => (i % 2 ? "full-attention" : "sliding-attention")),
    rope: { slidingDimensionCount: 128, fullDimensionCount: 256, slidingFreqBase: 10000, fullFreqBase: 1000000 },
    finalLogitSoftcap: 30,
  };
  return Object.assign(m, extra || {});
}

function modelTensors(layers, overrides) {
  const t = { "rope_freqs.weight": { type: "F32", dimensions: [128] }, "output_norm.weight": { type: "F32", dimensions: [512] },
    "output.weight": { type: "Q6_K", dimensions: [512, 1000] } };
  for (let l = 0; l < layers; l += 1) {
    for (const [n, typ, rows, k] of [["attn_q", "Q4_K", 1024, 512], ["attn_k", "Q4_K", 512, 512],
      ["attn_v", "Q6_K", 512, 512], ["attn_output", "Q4_K", 512, 1024], ["ffn_gate", "Q4_K", 1024, 512],
      ["ffn_up", "Q4_K", 1024, 512], ["ffn_down", "Q6_K", 512, 1024]]) {
      t[`blk.${l}.${n}.weight`] = { type: typ, dimensions: [k, rows] };
    }
    for (const n of ["attn_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm"]) {
      t[`blk.${l}.${n}.weight`] = { type: "F32", dimensions: [512] };
    }
    t[`blk.${l}.attn_q_norm.weight`] = { type: "F32", dimensions: [256] };
    t[`blk.${l}.attn_k_norm.weight`] = { type: "F32", dimensions: [256] };
    t[`blk.${l}.layer_output_scale.weight`] = { type: "F32", dimensions: [1] };
  }
  return Object.assign(t, overrides || {});
}

function modelSession(tensors, manifest) {
  const session = mockSession(tensors, ["wasm", "hip"]);
  session.tensorReader.owner = session;
  session.manifest = manifest;
  session.epsilon = 1e-6;
  session.readF32Tensor = async (name) => {
    const t = session.getTensor(name);
    const n = t.dimensions.reduce((a, b) => a * b, 1);
    return Float32Array.from({ length: n }, (_, i) => (name.endsWith("layer_output_scale.weight") ? 0.5 : 1 + i / 1000));
  };
  return session;
}

function stateOf(manifest, capacities, nextPosition) {
  const fullAttention = new Map();
  capacities.forEach((capacity, layer) => {
    const heads = manifest.headCountKv;
    fullAttention.set(layer, {
      key: Float32Array.from({ length: capacity * heads * 256 }, (_, i) => (i % 997) / 64 - 7),
      value: Float32Array.from({ length: capacity * heads * 256 }, (_, i) => (i % 991) / 32 - 15),
      keyLength: 256, valueLength: 256, headCountKv: heads, kind: layer % 2 ? "full" : "sliding",
      contextLength: 8192, capacity,
    });
  });
  return { fullAttention, contextLength: 8192, nextPosition };
}

async function segment() {
  const hip = require(HIP);
  const seg = require(path.join(__dirname, "..", "heliopause_amd", "napi", "hip", "segment-runner.js"));
  const log = [];
  const dev = fakeDevice(log);
  hip.setHipKernels(dev);
  const out = {};
  const tensors = modelTensors(2);
  const manifest = manifestOf(2);
  const session = modelSession(tensors, manifest);
  // what the device path covers
  out.support = seg.hipSegmentSupport(session, manifest, 0, 2);
  out.supportPle = seg.hipSegmentSupport(session, manifestOf(2, { perLayerEmbeddingLength: 256 }), 0, 2).reason;
  out.supportPleLength = seg.hipSegmentSupport(session, manifestOf(2, { perLayerEmbeddingLength: 100 }), 0, 2).reason;
  out.supportKvShared = seg.hipSegmentSupport(session, manifestOf(2, { layerHasKv: [true, false] }), 0, 2).reason;
  out.supportWidth = seg.hipSegmentSupport(session, manifestOf(2, { layerKeyLengths: [256, 512] }), 0, 2).reason;
  out.supportType = seg.hipSegmentSupport(modelSession(modelTensors(2, { "blk.1.ffn_up.weight": { type: "Q8_0",
    dimensions: [512, 1024] } }), manifest), manifest, 0, 2).reason;
  out.supportHidden = seg.hipSegmentSupport(session, manifestOf(2, { embeddingLength: 4352 }), 0, 2).reason;
  // the provider picks the device runner
  const engine = { createWasmModelRunner: () => ({ provider: "wasm", segmentRunner: async () => ({ provider: "wasm" }) }) };
  const runner = await hip.createHipModelRunner(engine).segmentRunner({ session, manifest, epsilon: 1e-6,
    segmentStartLayer: 0, segmentEndLayerExclusive: 2 });
  out.runnerProvider = [runner.provider, runner.segmentStartLayer, runner.segmentEndLayerExclusive];
  out.invalidSegment = await throws(() => seg.createHipSegmentRunner({ session, manifest, segmentStartLayer: 1,
    segmentEndLayerExclusive: 3 }));
  const fallback = await hip.createHipModelRunner(engine).segmentRunner({ session: modelSession(tensors,
    manifestOf(2, { perLayerEmbeddingLength: 256 })), manifest: manifestOf(2, { perLayerEmbeddingLength: 256 }),
  segmentStartLayer: 0, segmentEndLayerExclusive: 2 });
  out.fallbackProvider = [fallback.provider, fallback instanceof seg.HipSegmentRunner];
  // a state that already holds positions: its host caches go to the device rings
  const state = stateOf(manifest, [64, 8192], 300);
  const x = new Float32Array(3 * 512).fill(1);
  const r1 = await runner.runTokensHidden(x, Int32Array.of(300, 301, 302), state);
  const call = dev.calls[dev.calls.length - 1];
  out.lastOnly = [r1.hidden.length, call.rowStart, call.rowCount, call.position, call.tokenCount, call.inputLength];
  out.layer0 = Object.assign({}, call.layers[0], { attnQ: String(call.layers[0].attnQ), attnV: String(call.layers[0].attnV),
    keyCache: undefined, valueCache: undefined, attnNorm: undefined, attnQNorm: undefined, attnKNorm: undefined,
    postAttentionNorm: undefined, ffnNorm: undefined, postFfwNorm: undefined });
  out.layer0.attention = Object.assign({}, call.layers[0].attention, { ropeFreqFactors: String(call.layers[0].attention.ropeFreqFactors) });
  out.layer1Attention = Object.assign({}, call.layers[1].attention, { ropeFreqFactors: call.layers[1].attention.ropeFreqFactors !== 0n });
  // the imported ring: key slot 5, head 1, dim 3 and value slot 9, head 0, dim 200 of layer 1
  const ring = (ptr) => new Uint16Array(dev.buffers.get(ptr).buffer);
  const c1 = state.fullAttention.get(1);
  out.ringKey = [ring(call.layers[1].keyCache)[(1 * 8192 + 5) * 256 + 3], seg.f16Bits(c1.key[(5 * 2 + 1) * 256 + 3])];
  out.ringValue = [ring(call.layers[1].valueCache)[(0 * 8192 + 9) * 256 + 200], seg.f16Bits(c1.value[(200 * 2 + 0) * 8192 + 9])];
  out.norm0 = Array.from(new Float32Array(dev.buffers.get(call.layers[0].attnNorm).buffer).slice(0, 3));
  // a state seen first at position 0 has zeroed rings (no host copy)
  const fresh = stateOf(manifest, [64, 8192], 0);
  await runner.runTokensHidden(new Float32Array(512), Int32Array.of(0), fresh);
  const c2 = dev.calls[dev.calls.length - 1];
  out.freshRingZero = ring(c2.layers[1].keyCache).every((v) => v === 0);
  out.freshRows = [c2.rowStart, c2.rowCount];
  // a middle segment returns every row
  const middle = await seg.createHipSegmentRunner({ session, manifest, segmentStartLayer: 0, segmentEndLayerExclusive: 1 });
  const rm = await middle.runTokensHidden(x, Int32Array.of(10, 11, 12), stateOf(manifest, [64], 0));
  out.middleRows = [rm.hidden.length, rm.hidden[0], rm.hidden[512 * 2]];
  out.nonConsecutive = await throws(() => runner.runTokensHidden(x, Int32Array.of(5, 7, 8), state));
  out.outside = await throws(() => runner.runTokensHidden(new Float32Array(512), Int32Array.of(8192), state));
  out.notCausal = await throws(() => runner.runTokensHidden(new Float32Array(512), Int32Array.of(1), state,
    { attentionCausal: false }));
  out.badShape = await throws(() => runner.runTokenHidden(x, Int32Array.of(1, 2, 3), state));
  // the head on the device
  const tok = await runner.runToken(new Float32Array(512), Int32Array.of(303), state);
  const headCall = dev.calls[dev.calls.length - 1];
  const layersCall = dev.calls[dev.calls.length - 2];
  out.runToken = { top: tok.topTokens, selected: tok.selectedTokenId, topK: headCall.topK, softcap: headCall.softcap,
    readOutput: layersCall.readOutput, outputNorm: layersCall.bufs.outputNorm !== 0n,
    headInput: headCall.dInput === String(layersCall.bufs.output) };
  out.middleRunToken = await throws(() => middle.runToken(new Float32Array(512), Int32Array.of(1), state));
  // release frees every device buffer the runners allocated
  runner.release();
  middle.release();
  out.allocs = log.filter((l) => l.startsWith("alloc")).length;
  out.frees = log.filter((l) => l === "free").length;
  out.leftBuffers = dev.buffers.size;
  out.afterRelease = await throws(() => runner.runTokensHidden(new Float32Array(512), Int32Array.of(1), state));
  // the per-layer input step: layer 1 of a 3-layer model, 2 tokens, P = 256
  const pleTensors = modelTensors(3);
  for (let l = 0; l < 3; l += 1) {
    pleTensors[`blk.${l}.inp_gate.weight`] = { type: "Q6_K", dimensions: [512, 256] };
    pleTensors[`blk.${l}.proj.weight`] = { type: "Q4_K", dimensions: [256, 512] };
    pleTensors[`blk.${l}.post_norm.weight`] = { type: "F32", dimensions: [512] };
  }
  const pleManifest = manifestOf(3, { perLayerEmbeddingLength: 256 });
  const pleSession = modelSession(pleTensors, pleManifest);
  const pleRunner = await seg.createHipSegmentRunner({ session: pleSession, manifest: pleManifest,
    segmentStartLayer: 1, segmentEndLayerExclusive: 2 });
  const pleState = stateOf(pleManifest, [64, 8192, 64], 0);
  const pli = Float32Array.from({ length: 3 * 2 * 256 }, (_, i) => i);
  await pleRunner.runTokensHidden(new Float32Array(2 * 512), Int32Array.of(4, 5), pleState, { perLayerInputs: pli });
  const pc = dev.calls[dev.calls.length - 1];
  const rows = new Float32Array(dev.buffers.get(pc.layers[0].perLayerInput).buffer);
  out.ple = { hasGate: pc.layers[0].inpGate !== undefined && pc.layers[0].proj !== undefined,
    postNorm: pc.layers[0].postNorm !== undefined, first: rows[0], last: rows[2 * 256 - 1] };
  await pleRunner.runTokensHidden(new Float32Array(512), Int32Array.of(6), pleState);
  out.pleSkipped = dev.calls[dev.calls.length - 1].layers[0].perLayerInput === undefined;
  out.pleShape = await throws(() => pleRunner.runTokensHidden(new Float32Array(512), Int32Array.of(7), pleState,
    { perLayerInputs: new Float32Array(10) }));
  pleRunner.release();
  process.stdout.write(JSON.stringify(out, (key, v) => (typeof v === "bigint" ? String(v) : v)));
}

/* The device segment runner over a GGUF file (GPU): case.json gives the
 * manifest, the state's caches come from cache_<layer>_{key,value}.bin (the
 * host layout of updateFullAttentionCache), x.bin / x2.bin the two tokens'
 * rows.  Writes out_hidden.bin (runTokensHidden at `position`) and returns
 * runToken's top-k at position + 1 and the ms per token of both calls. */
async function segmentGpu(dir) {
  const hip = require(HIP);
  const c = JSON.parse(fs.readFileSync(path.join(dir, "case.json"), "utf8"));
  const session = fileSession(path.join(dir, "model.gguf"));
  const kernels = require(path.join(__dirname, "..", "heliopause_amd", "napi", "hip-kernels.js"));
  const fd = fs.openSync(path.join(dir, "model.gguf"), "r");
  session.readF32Tensor = async (name) => {
    const t = session.getTensor(name);
    const b = Buffer.alloc(t.byteLength);
    fs.readSync(fd, b, 0, t.byteLength, Number(t.dataOffset));
    return new Float32Array(b.buffer, b.byteOffset, t.byteLength / 4).slice();
  };
  session.epsilon = c.epsilon;
  const manifest = {
    blockCount: c.layers, embeddingLength: c.hidden, headCount: c.headCount, headCountKv: c.headCountKv,
    layerHeadCountKv: [], keyLength: 256, valueLength: 256, layerKeyLengths: [], layerValueLengths: [],
    layerHasKv: Array(c.layers).fill(true), layerValueProjectionModes: Array(c.layers).fill("separate"),
    kvSourceLayers: [], slidingWindow: c.slidingWindow, perLayerEmbeddingLength: 0, layerKinds: c.kinds,
    rope: c.rope, contextLength: c.contextLength,
  };
  session.manifest = manifest;
  const fullAttention = new Map();
  for (let l = 0; l < c.layers; l += 1) {
    fullAttention.set(l, {
      key: readF32(path.join(dir, `cache_${l}_key.bin`)).slice(),
      value: readF32(path.join(dir, `cache_${l}_value.bin`)).slice(),
      keyLength: 256, valueLength: 256, headCountKv: c.headCountKv,
      kind: c.kinds[l] === "sliding-attention" ? "sliding" : "full", contextLength: c.contextLength,
      capacity: c.capacities[l],
    });
  }
  const state = { fullAttention, contextLength: c.contextLength, nextPosition: c.position };
  const engine = { createWasmModelRunner: () => ({ provider: "wasm", segmentRunner: async () => ({ provider: "wasm" }) }) };
  hip.registerHipExecutionProvider(session);
  const t0 = Date.now();
  const runner = await hip.createHipModelRunner(engine).segmentRunner({ session, state, manifest,
    epsilon: c.epsilon, segmentStartLayer: 0, segmentEndLayerExclusive: c.layers });
  const createMs = Date.now() - t0;
  const x = readF32(path.join(dir, "x.bin")).slice();
  const r = await runner.runTokensHidden(x, Int32Array.of(c.position), state);
  writeF32(path.join(dir, "out_hidden.bin"), r.hidden);
  const tok = await runner.runToken(readF32(path.join(dir, "x2.bin")).slice(), Int32Array.of(c.position + 1), state,
    { topK: c.topK });
  // ms per token: the same state, later positions (its rings keep filling)
  const time = async (fn) => {
    await fn(c.position + 2);
    const start = process.hrtime.bigint();
    for (let i = 0; i < c.steps; i += 1) {
      await fn(c.position + 3 + i);
    }
    return Number(process.hrtime.bigint() - start) / 1e6 / c.steps;
  };
  const hiddenMs = await time((p) => runner.runTokensHidden(x, Int32Array.of(p), state));
  const tokenMs = await time((p) => runner.runToken(x, Int32Array.of(p), state, { topK: c.topK }));
  runner.release();
  hip.shutdownHipExecutionProvider(session);
  fs.closeSync(fd);
  session.close();
  process.stdout.write(JSON.stringify({ provider: runner.provider, top: tok.topTokens, selected: tok.selectedTokenId,
    hiddenMs, tokenMs, createMs, stats: kernels.hipResidentWeightStats() }));
}

/* f16 bits of the f32 values whose bits are on stdin (JSON array). */
function f16() {
  const seg = require(path.join(__dirname, "..", "heliopause_amd", "napi", "hip", "segment-runner.js"));
  const bits = JSON.parse(fs.readFileSync(0, "utf8"));
  const f = new Float32Array(Uint32Array.from(bits).buffer);
  process.stdout.write(JSON.stringify(Array.from(f, (v) => seg.f16Bits(v))));
}

/* shutdownHipExecutionProvider while an upload is pending: the late handle
 * is released, not cached. */
async function race() {
  const hip = require(HIP);
  const log = [];
  const k = fakeKernels(log);
  let resolveCreate;
  const create = k.createHipQuantizedWeightHandle;
  k.createHipQuantizedWeightHandle = (type, bytes, inputSize, rowCount) => new Promise((resolve) => {
    resolveCreate = () => resolve({ handle: 99n, type, byteLength: 64, rowCount, inputSize, released: false });
  });
  hip.setHipKernels(k);
  const session = mockSession({ "blk.0.attn_q.weight": { type: "Q4_K", dimensions: [256, 8] } }, ["hip"]);
  session.tensorReader.owner = session;
  hip.registerHipExecutionProvider(session);
  const pending = hip.readHipWeightHandle(session, "blk.0.attn_q.weight", "Q4_K", 256, 8);
  while (!resolveCreate) {
    await new Promise((resolve) => setTimeout(resolve, 1));
  }
  hip.shutdownHipExecutionProvider(session);
  resolveCreate();
  const got = await pending;
  k.createHipQuantizedWeightHandle = create;
  const after = await hip.readHipWeightHandle(session, "blk.0.attn_q.weight", "Q4_K", 256, 8);
  process.stdout.write(JSON.stringify({ got: String(got), log, stats: session.statsProviders.hip(),
    secondCall: after ? String(after.handle) : "undefined" }));
}

const mode = process.argv[2];
const jobs = { dispatch, nogpu, segment, race, f16: async () => f16() };
const job = jobs[mode] ? jobs[mode]() : mode === "segment-gpu" ? segmentGpu(process.argv[3]) : layer(process.argv[3]);
job.catch((error) => {
  process.stderr.write(`${error.stack || error}\n`);
  process.exit(1);
});
