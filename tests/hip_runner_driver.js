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

const mode = process.argv[2];
const job = mode === "dispatch" ? dispatch() : mode === "nogpu" ? nogpu() : layer(process.argv[3]);
job.catch((error) => {
  process.stderr.write(`${error.stack || error}\n`);
  process.exit(1);
});
