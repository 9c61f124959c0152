"use strict";
// Drives heliopause_amd/napi/hip-kernels.js from Node for the N-API tests.
//   node napi_driver.js api            -> JSON of the API-level checks that need no GPU
//   node napi_driver.js run <dir>      -> reads case.json + *.bin from <dir>, runs the
//                                         projections through the addon, writes out_*.bin
//   node napi_driver.js gguf <file> <maxArraySample> [completeKey...]
//                                      -> the parsed file as JSON (bigints as strings,
//                                         like serializeGgufMetadata, gguf.ts:246-259)
//   node napi_driver.js ggufrun <dir>  -> loads <dir>/model.gguf through HipGgufWeights,
//                                         projects <dir>/x.bin with every handle
const fs = require("fs");
const path = require("path");
const hip = require(path.join(__dirname, "..", "heliopause_amd", "napi", "hip-kernels.js"));

async function throws(fn) {
  try {
    await fn();
    return "";
  } catch (error) {
    return error.message;
  }
}

async function api() {
  const fake = { handle: 1n, type: "Q4_K", byteLength: 144, rowCount: 1, inputSize: 256, released: false };
  const released = Object.assign({}, fake, { released: true });
  const out = {
    exports: Object.keys(hip).sort(),
    support: await hip.checkHipSupport(),
    typeIds: ["Q4_K", "Q5_K", "Q6_K", "IQ4_XS", "Q8_0", "Q4_0", "F16"].map((t) => hip.quantizedTypeId(t) || 0),
    unknownType: String(await hip.createHipQuantizedWeightHandle("F16", new Uint8Array(4), 256, 1)),
    zeroShape: await throws(() => hip.createHipQuantizedWeightHandle("Q4_K", new Uint8Array(0), 0, 1)),
    scaleShape: await throws(() => hip.createHipQuantizedWeightHandle("Q6_K", new Uint8Array(210), 100, 1)),
    multiOne: String(await hip.matMulQuantizedHipResidentMulti([fake], new Float32Array(256), 256, 1)),
    multiFive: String(await hip.matMulQuantizedHipResidentMulti([fake, fake, fake, fake, fake], new Float32Array(256), 256, 1)),
    handleShape: await throws(() => hip.matMulQuantizedHipResident(fake, new Float32Array(256), 256, 2, 1)),
    inputShape: await throws(() => hip.matMulQuantizedHipResident(fake, new Float32Array(255), 256, 1, 1)),
    releasedHandle: await throws(() => hip.matMulQuantizedHipResident(released, new Float32Array(256), 256, 1, 1)),
    multiShape: await throws(() =>
      hip.matMulQuantizedHipResidentMulti([fake, Object.assign({}, fake, { inputSize: 512 })], new Float32Array(256), 256, 1),
    ),
    assertShape: await throws(() => hip.assertHipOk(1, "k")),
    assertType: await throws(() => hip.assertHipOk(3, "k")),
    sampling: hip.resolveGenerationSamplingOptions(),
    samplingGreedy: hip.resolveGenerationSamplingOptions({ doSample: false, topK: 64 }).logitsTopK,
    samplingTopK: hip.resolveGenerationSamplingOptions({ topK: 64.9 }).topK,
    samplingBadTemp: await throws(() => hip.resolveGenerationSamplingOptions({ temperature: -1 })),
    samplingBadTopP: await throws(() => hip.resolveGenerationSamplingOptions({ topP: 1.1 })),
    samplingState: Array.from(hip.createHipSamplingState(-1)),
  };
  process.stdout.write(JSON.stringify(out));
}

function readF32(file) {
  const b = fs.readFileSync(file);
  return new Float32Array(b.buffer, b.byteOffset, b.byteLength / 4);
}

async function run(dir) {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, "case.json"), "utf8"));
  const support = await hip.checkHipSupport();
  if (!support.available) {
    throw new Error(`HIP runner unavailable: ${JSON.stringify(support)}`);
  }
  const x = readF32(path.join(dir, "x.bin"));
  const handles = [];
  for (const w of spec.weights) {
    const bytes = new Uint8Array(fs.readFileSync(path.join(dir, w.file)));
    handles.push(await hip.createHipQuantizedWeightHandle(w.type, bytes, spec.inputSize, w.rows));
  }
  const stats = hip.hipResidentWeightStats();
  const single = await hip.matMulQuantizedHipResident(handles[0], x, spec.inputSize, spec.weights[0].rows, spec.columns);
  fs.writeFileSync(path.join(dir, "out_single.bin"), Buffer.from(single.buffer, single.byteOffset, single.byteLength));
  const multi = await hip.matMulQuantizedHipResidentMulti(handles.slice(0, 3), x, spec.inputSize, spec.columns);
  multi.forEach((o, i) => fs.writeFileSync(path.join(dir, `out_multi${i}.bin`), Buffer.from(o.buffer, o.byteOffset, o.byteLength)));
  // gate/up pair (weights 3 and 4) and the head (weight 5) run concurrently on the libuv pool
  const [geglu, top] = await Promise.all([
    hip.matMulGegluHipResident(handles[3], handles[4], x, spec.inputSize, spec.columns),
    hip.matMulQuantizedHipResidentTopK(handles[5], x, spec.inputSize, spec.columns, spec.topK, spec.softcap),
  ]);
  fs.writeFileSync(path.join(dir, "out_geglu.bin"), Buffer.from(geglu.buffer, geglu.byteOffset, geglu.byteLength));
  fs.writeFileSync(path.join(dir, "out_topk.json"), JSON.stringify(top));
  // head + top-k + sampling with a seeded state, twice (the state advances)
  const sampling = hip.resolveGenerationSamplingOptions({ temperature: 0.8, topP: 0.9, topK: 40, seed: spec.seed });
  const state = hip.createHipSamplingState(sampling.seed);
  const sampled = [];
  for (let i = 0; i < 2; i += 1) {
    sampled.push(await hip.matMulQuantizedHipResidentTopKSample(handles[5], x, spec.inputSize, spec.columns, sampling, state, spec.softcap));
  }
  fs.writeFileSync(path.join(dir, "out_sample.json"), JSON.stringify({ sampled, state: state[0] }));
  const mismatch = await throws(() => hip.matMulQuantizedHipResident(handles[0], x, spec.inputSize + 256, spec.weights[0].rows, spec.columns));
  handles.forEach((h) => hip.releaseHipQuantizedWeightHandle(h));
  const after = hip.hipResidentWeightStats();
  process.stdout.write(JSON.stringify({ residentBefore: stats.residentBytes, residentAfter: after.residentBytes, handlesAfter: after.handleCount, mismatch }));
}

function serialize(value) {
  return JSON.stringify(value, (key, v) => (typeof v === "bigint" ? v.toString() : v));
}

async function gguf(file, maxArraySample, keys) {
  const f = hip.openHipGgufFile(file, { maxArraySample: Number(maxArraySample), completeArrayKeys: keys });
  try {
    process.stdout.write(serialize(f.metadata));
  } finally {
    f.close();
  }
}

async function ggufRun(dir) {
  const spec = JSON.parse(fs.readFileSync(path.join(dir, "case.json"), "utf8"));
  const x = readF32(path.join(dir, "x.bin"));
  const f = hip.openHipGgufFile(path.join(dir, "model.gguf"));
  const weights = new hip.HipGgufWeights(f);
  const names = f.metadata.tensors.map((t) => t.name);
  // a single-tensor request and a batch racing it share one upload
  const [first, all] = await Promise.all([weights.handle(names[0]), weights.upload(names)]);
  const again = await weights.handle(names[0]);
  const result = { supported: [], unsupported: [], sameHandle: first === again && first === all.get(names[0]) };
  for (const name of names) {
    const h = all.get(name);
    if (!h) {
      result.unsupported.push(name);
      continue;
    }
    result.supported.push(name);
    const out = await hip.matMulQuantizedHipResident(h, x.subarray(0, h.inputSize * spec.columns), h.inputSize, h.rowCount, spec.columns);
    fs.writeFileSync(path.join(dir, `out_${name}.bin`), Buffer.from(out.buffer, out.byteOffset, out.byteLength));
  }
  result.hits = weights.hits;
  result.misses = weights.misses;
  result.bytes = weights.bytes;
  weights.release();
  result.handlesAfter = hip.hipResidentWeightStats().handleCount;
  f.close();
  process.stdout.write(JSON.stringify(result));
}

const mode = process.argv[2];
const job = mode === "api" ? api()
  : mode === "gguf" ? gguf(process.argv[3], process.argv[4], process.argv.slice(5))
  : mode === "ggufrun" ? ggufRun(process.argv[3])
  : run(process.argv[3]);
job.catch((error) => {
  process.stderr.write(`${error.stack || error}\n`);
  process.exit(1);
});
