"use strict";
/*
 * hip/segment-runner.js -- the HIP runner's SegmentRunner
 * (packages/engine/src/runner/segment-runner.ts:18-34) with device-resident
 * state, as the WebGPU runner keeps its own (webgpu/segment-runner.ts:1123-
 * 1290): the layers of the segment run in HBM through
 * hp_hip_decode_layers_device, one call per runTokensHidden, and only the
 * input rows go in and the result rows come back.
 *
 *   WasmSegmentRunner (wasm/segment-runner.ts:63-207)   HipSegmentRunner
 *     runTokensHidden / runTokenHidden                   same signatures, same rows returned
 *     sliding-ring chunking (slidingRingChunkTokenCount) inside the device call
 *   forwardAttentionLayer + forwardFfn (wasm/layers.ts:161-473)
 *                                                        hp_hip_decode_layers_device
 *   WebGPU runToken (webgpu/segment-runner.ts:1123-1158) runToken: the segment,
 *     the output norm and the head on the device, top-k (and a sampled token)
 *     read back (forwardOutput, wasm/layers.ts:381-416)
 *
 * Per InferenceState the runner keeps f16 KV rings in HBM, one per layer,
 * [head_count_kv][capacity][256] with the capacity of the state's cache for
 * that layer (state.fullAttention); a state that already holds positions
 * when the runner first sees it has its host caches copied in.  The host
 * caches are not written back: the state's keys and values live on the
 * device, as the WebGPU runner's do.
 *
 * createHipSegmentRunner returns undefined (the caller keeps the WASM
 * runner) when the GPU or the addon is missing or a layer is outside what
 * the device path covers: every layer with its own KV, key and value width
 * 256, query heads a multiple of the KV heads (at most 8 per KV head),
 * Q4_K/Q6_K projections (inp_gate and proj of the per-layer input step
 * included, applyPerLayerInput layers.ts:475-521), F32 norms, hidden size a
 * multiple of 256 up to 4096.  A run given options.perLayerInputs (the
 * [layer][token][P] array of preparePerLayerInputs) runs that step in every
 * layer; a run without it skips it, as forwardAttentionLayer does.
 */

const acceleration = require("./acceleration.js");

const HEAD_DIM = 256;
const MAX_HIDDEN = 4096;
const MAX_GROUP = 8;
const QUANTIZED = new Set(["Q4_K", "Q6_K"]);
const NORMS = {
  attnNorm: "attn_norm",
  attnQNorm: "attn_q_norm",
  attnKNorm: "attn_k_norm",
  postAttentionNorm: "post_attention_norm",
  ffnNorm: "ffn_norm",
  postFfwNorm: "post_ffw_norm",
};

function tensorInfo(session, name) {
  try {
    return session.getTensor(name);
  } catch (error) {
    return undefined;
  }
}

function layerKind(manifest, layer) {
  return manifest.layerKinds[layer] || "sliding-attention";
}

function valueShared(manifest, layer) {
  return manifest.layerValueProjectionModes && manifest.layerValueProjectionModes[layer] === "shared-with-key";
}

/* Whether layers [start, end) run on the device path; {supported, reason}. */
function hipSegmentSupport(session, manifest, start, end) {
  const hidden = manifest.embeddingLength;
  if (hidden % 256 !== 0 || hidden > MAX_HIDDEN) {
    return { supported: false, reason: `hidden size ${hidden}` };
  }
  const ple = manifest.perLayerEmbeddingLength > 0;
  if (ple && manifest.perLayerEmbeddingLength % 256 !== 0) {
    return { supported: false, reason: `per-layer input length ${manifest.perLayerEmbeddingLength}` };
  }
  for (let layer = start; layer < end; layer += 1) {
    if (manifest.layerHasKv[layer] !== true) {
      return { supported: false, reason: `layer ${layer} reads another layer's KV` };
    }
    const keyLength = manifest.layerKeyLengths[layer] || manifest.keyLength;
    const valueLength = manifest.layerValueLengths[layer] || manifest.valueLength;
    if (keyLength !== HEAD_DIM || valueLength !== HEAD_DIM) {
      return { supported: false, reason: `layer ${layer} head width ${keyLength}/${valueLength}` };
    }
    const kvHeads = (manifest.layerHeadCountKv && manifest.layerHeadCountKv[layer]) || manifest.headCountKv;
    if (manifest.headCount % kvHeads !== 0 || manifest.headCount / kvHeads > MAX_GROUP) {
      return { supported: false, reason: `layer ${layer} heads ${manifest.headCount}/${kvHeads}` };
    }
    const projections = ["attn_q", "attn_k", "attn_output", "ffn_gate", "ffn_up", "ffn_down"];
    if (!valueShared(manifest, layer)) {
      projections.push("attn_v");
    }
    if (ple) {
      projections.push("inp_gate", "proj");
      const post = tensorInfo(session, `blk.${layer}.post_norm.weight`);
      if (!post || post.type !== "F32") {
        return { supported: false, reason: `blk.${layer}.post_norm.weight` };
      }
    }
    for (const name of projections) {
      const tensor = tensorInfo(session, `blk.${layer}.${name}.weight`);
      if (!tensor || !QUANTIZED.has(tensor.type)) {
        return { supported: false, reason: `blk.${layer}.${name}.weight type ${tensor ? tensor.type : "missing"}` };
      }
    }
    for (const name of Object.values(NORMS)) {
      const tensor = tensorInfo(session, `blk.${layer}.${name}.weight`);
      if (!tensor || tensor.type !== "F32") {
        return { supported: false, reason: `blk.${layer}.${name}.weight` };
      }
    }
  }
  return { supported: true };
}

/* f16 bits of an f32 value, round to nearest even (the device caches'
 * entries; the host caches are f32). */
const f32Scratch = new Float32Array(1);
const u32Scratch = new Uint32Array(f32Scratch.buffer);
function f16Bits(value) {
  f32Scratch[0] = value;
  const x = u32Scratch[0];
  const sign = (x >>> 16) & 0x8000;
  const exponent = (x >>> 23) & 0xff;
  let mantissa = x & 0x7fffff;
  if (exponent === 0xff) {
    return sign | 0x7c00 | (mantissa !== 0 ? 0x200 : 0);
  }
  const e = exponent - 127 + 15;
  if (e >= 0x1f) {
    return sign | 0x7c00;
  }
  if (e <= 0) {
    if (e < -10) {
      return sign;
    }
    mantissa |= 0x800000;
    const shift = 14 - e;
    let h = mantissa >>> shift;
    const rest = mantissa & ((1 << shift) - 1);
    const half = 1 << (shift - 1);
    if (rest > half || (rest === half && (h & 1) !== 0)) {
      h += 1;
    }
    return sign | h;
  }
  let h = (e << 10) | (mantissa >>> 13);
  const rest = mantissa & 0x1fff;
  if (rest > 0x1000 || (rest === 0x1000 && (h & 1) !== 0)) {
    h += 1;
  }
  return sign | h;
}

/* The host cache of updateFullAttentionCache (layers.ts:887-911: key
 * [slot][head][dim], value [dim][head][slot], f32) as the device ring's f16
 * [head][slot][dim] rows. */
function deviceRingFromHost(cache) {
  const heads = cache.headCountKv;
  const capacity = cache.capacity;
  const key = new Uint16Array(heads * capacity * HEAD_DIM);
  const value = new Uint16Array(heads * capacity * HEAD_DIM);
  for (let slot = 0; slot < capacity; slot += 1) {
    for (let head = 0; head < heads; head += 1) {
      const row = (head * capacity + slot) * HEAD_DIM;
      for (let dim = 0; dim < HEAD_DIM; dim += 1) {
        key[row + dim] = f16Bits(cache.key[(slot * heads + head) * cache.keyLength + dim]);
        value[row + dim] = f16Bits(cache.value[(dim * heads + head) * capacity + slot]);
      }
    }
  }
  return { key, value };
}

/* Positions of the tokens: the device call takes the first and counts up. */
function firstPosition(positions, tokenCount, contextLength) {
  if (positions.length !== tokenCount) {
    throw new Error(`HIP segment positions shape mismatch: ${positions.length} for ${tokenCount} tokens`);
  }
  for (let token = 0; token < tokenCount; token += 1) {
    const position = positions[token];
    if (position < 0 || position >= contextLength) {
      throw new Error(`Position ${position} is outside context length ${contextLength}`);
    }
    if (position !== positions[0] + token) {
      throw new Error("The HIP segment runner takes consecutive positions.");
    }
  }
  return positions[0];
}

class HipSegmentRunner {
  constructor(options, layers, owned, kernels) {
    this.provider = "hip";
    this.session = options.session;
    this.manifest = options.manifest || options.session.manifest;
    this.epsilon = options.epsilon !== undefined ? options.epsilon : options.session.epsilon;
    this.segmentStartLayer = options.segmentStartLayer;
    this.segmentEndLayerExclusive = options.segmentEndLayerExclusive;
    this.kernels = kernels;
    this.layers = layers; // per layer: handles, norm buffers, scale, attention parameters (no state)
    this.owned = owned; // device buffers of the weights' norms and RoPE factors
    this.states = new WeakMap();
    this.stateBuffers = [];
    this.queue = Promise.resolve();
    this.output = undefined; // output_norm buffer and head handle (runToken)
    this.released = false;
  }

  /* Device rings and row buffers of `state` (created on first use). */
  stateFor(state, tokenCount) {
    const k = this.kernels;
    let s = this.states.get(state);
    if (!s) {
      s = { caches: [], hidden: undefined, output: undefined, rows: 0, position: k.deviceAlloc(16) };
      this.stateBuffers.push(s.position);
      for (const layer of this.layers) {
        const cache = state.fullAttention.get(layer.layer);
        if (!cache) {
          throw new Error(`Missing full-attention cache for layer ${layer.layer}`);
        }
        if (cache.headCountKv !== layer.headCountKv) {
          throw new Error(`KV heads of layer ${layer.layer}: cache ${cache.headCountKv}, model ${layer.headCountKv}`);
        }
        const bytes = cache.headCountKv * cache.capacity * HEAD_DIM * 2;
        const ring = { capacity: cache.capacity, key: k.deviceAlloc(bytes), value: k.deviceAlloc(bytes) };
        this.stateBuffers.push(ring.key, ring.value);
        if (state.nextPosition > 0) {
          const host = deviceRingFromHost(cache);
          k.copyToDevice(ring.key, host.key);
          k.copyToDevice(ring.value, host.value);
        }
        s.caches.push(ring);
      }
      this.states.set(state, s);
    }
    if (s.rows < tokenCount) {
      const bytes = tokenCount * this.manifest.embeddingLength * 4;
      for (const ptr of [s.hidden, s.output]) {
        if (ptr) {
          k.deviceFree(ptr);
          this.stateBuffers.splice(this.stateBuffers.indexOf(ptr), 1);
        }
      }
      s.hidden = k.deviceAlloc(bytes);
      s.output = k.deviceAlloc(bytes);
      this.stateBuffers.push(s.hidden, s.output);
      s.rows = tokenCount;
    }
    return s;
  }

  /* The layer objects of one call: the state's rings, and with the
   * per-layer inputs ([layer][token][P], every layer of the model) this
   * segment's rows of them in a device buffer, one block per layer. */
  descriptors(s, perLayerInputs, tokenCount) {
    const P = this.manifest.perLayerEmbeddingLength;
    let pli;
    if (perLayerInputs && P > 0) {
      const start = this.segmentStartLayer;
      const count = this.segmentEndLayerExclusive - start;
      if (perLayerInputs.length !== this.manifest.blockCount * tokenCount * P) {
        throw new Error(`Per-layer input shape mismatch: ${perLayerInputs.length}`);
      }
      const bytes = count * tokenCount * P * 4;
      if (!s.pli || s.pliBytes < bytes) {
        if (s.pli) {
          this.kernels.deviceFree(s.pli);
          this.stateBuffers.splice(this.stateBuffers.indexOf(s.pli), 1);
        }
        s.pli = this.kernels.deviceAlloc(bytes);
        s.pliBytes = bytes;
        this.stateBuffers.push(s.pli);
      }
      this.kernels.copyToDevice(s.pli, perLayerInputs.subarray(start * tokenCount * P, (start + count) * tokenCount * P));
      pli = s.pli;
    }
    return this.layers.map((layer, index) => {
      const d = Object.assign({}, layer.descriptor, {
        keyCache: s.caches[index].key,
        valueCache: s.caches[index].value,
        attention: Object.assign({}, layer.descriptor.attention, { capacity: s.caches[index].capacity }),
      });
      if (pli !== undefined && layer.ple) {
        Object.assign(d, layer.ple, { perLayerInput: pli + BigInt(index * tokenCount * P * 4) });
      }
      return d;
    });
  }

  /* Calls on one runner run one at a time: they share its row buffers. */
  serial(fn) {
    const run = this.queue.then(fn, fn);
    this.queue = run.then(() => undefined, () => undefined);
    return run;
  }

  async runTokensHidden(inputHidden, positions, state, options) {
    const opts = options || {};
    if (this.released) {
      throw new Error("The HIP segment runner was released.");
    }
    if (opts.attentionCausal === false) {
      throw new Error("The HIP segment runner runs causal attention only.");
    }
    const hiddenSize = this.manifest.embeddingLength;
    const tokenCount = inputHidden.length / hiddenSize;
    if (!Number.isInteger(tokenCount) || tokenCount < 1) {
      throw new Error(`HIP segment input shape mismatch: ${inputHidden.length}`);
    }
    const position = firstPosition(positions, tokenCount, state.contextLength);
    if (this.segmentEndLayerExclusive === this.segmentStartLayer) {
      return { hidden: inputHidden };
    }
    // the model's last layer returns only the last token's row
    // (forwardAttentionLayer, layers.ts:375-377; the chunked path's lastHidden)
    const lastOnly = this.segmentEndLayerExclusive === this.manifest.blockCount && tokenCount > 1;
    return this.serial(async () => {
      const s = this.stateFor(state, tokenCount);
      const hidden = await this.kernels.runDecodeLayers(this.descriptors(s, opts.perLayerInputs, tokenCount),
        tokenCount, hiddenSize,
        { hidden: s.hidden, position: s.position, outputNorm: 0n, output: 0n }, inputHidden, position, false,
        lastOnly ? tokenCount - 1 : 0, lastOnly ? 1 : tokenCount);
      return { hidden };
    });
  }

  async runTokenHidden(inputHidden, positions, state, options) {
    if (inputHidden.length !== this.manifest.embeddingLength) {
      throw new Error(`HIP segment input shape mismatch: ${inputHidden.length}`);
    }
    return this.runTokensHidden(inputHidden, positions, state, options);
  }

  /* The output norm and head of a segment that ends at the model's last
   * layer (forwardOutput, layers.ts:381-416). */
  async outputParts() {
    if (!this.output) {
      const session = this.session;
      const norm = await session.readF32Tensor("output_norm.weight");
      const name = session.tensorReader.metadata.tensors.some((tensor) => tensor.name === "output.weight")
        ? "output.weight"
        : "token_embd.weight";
      const tensor = session.getTensor(name);
      const head = await acceleration.readHipWeightHandle(session, name, tensor.type, tensor.dimensions[0],
        tensor.dimensions[1]);
      if (!head) {
        throw new Error(`The HIP runner cannot hold ${name} (${tensor.type}).`);
      }
      const normBuffer = this.kernels.deviceAlloc(norm.byteLength);
      this.owned.push(normBuffer);
      this.kernels.copyToDevice(normBuffer, norm);
      this.output = { norm: normBuffer, head };
    }
    return this.output;
  }

  /* One token through the segment, the output norm and the head on the
   * device (the WebGPU runner's runToken, webgpu/segment-runner.ts:1123-1158):
   * {topTokens} (options.topK, default 10), or with options.sampling
   * (resolveGenerationSamplingOptions) and options.samplingState
   * (createHipSamplingState) also {selectedTokenId, distribution}. */
  async runToken(inputHidden, positions, state, options) {
    const opts = options || {};
    if (this.segmentEndLayerExclusive !== this.manifest.blockCount) {
      throw new Error("runToken needs a segment that ends at the model's last layer.");
    }
    const hiddenSize = this.manifest.embeddingLength;
    if (inputHidden.length !== hiddenSize) {
      throw new Error(`HIP segment input shape mismatch: ${inputHidden.length}`);
    }
    const position = firstPosition(positions, 1, state.contextLength);
    const parts = await this.outputParts();
    return this.serial(async () => {
      const s = this.stateFor(state, 1);
      await this.kernels.runDecodeLayers(this.descriptors(s, opts.perLayerInputs, 1), 1, hiddenSize,
        { hidden: s.hidden, position: s.position, outputNorm: parts.norm, output: s.output }, inputHidden, position,
        true, 0, 0);
      const softcap = this.manifest.finalLogitSoftcap;
      if (opts.sampling) {
        const [column] = await this.kernels.headTopKDevice(parts.head, s.output, hiddenSize, 1, opts.sampling.topK,
          softcap, opts.sampling, opts.samplingState);
        return {
          selectedTokenId: column.token,
          topTokens: column.distribution.map((c) => ({ id: c.id, value: c.value })),
          distribution: column.distribution,
        };
      }
      const [top] = await this.kernels.headTopKDevice(parts.head, s.output, hiddenSize, 1,
        opts.topK === undefined ? 10 : opts.topK, softcap);
      return { selectedTokenId: top.length > 0 ? top[0].id : undefined, topTokens: top };
    });
  }

  /* Frees the runner's device buffers (weights stay in the session cache). */
  release() {
    if (this.released) {
      return;
    }
    this.released = true;
    for (const ptr of this.stateBuffers.concat(this.owned)) {
      this.kernels.deviceFree(ptr);
    }
    this.stateBuffers = [];
    this.owned = [];
    this.states = new WeakMap();
  }
}

/* The device segment runner for ModelSegmentRunnerOptions
 * (runner/model-runner.ts:22-29), or undefined when it does not apply. */
async function createHipSegmentRunner(options) {
  const kernels = acceleration.hipKernels();
  const session = options.session;
  if (typeof kernels.runDecodeLayers !== "function" || !session) {
    return undefined;
  }
  const manifest = options.manifest || session.manifest;
  const start = options.segmentStartLayer === undefined ? 0 : options.segmentStartLayer;
  const end = options.segmentEndLayerExclusive === undefined ? manifest.blockCount : options.segmentEndLayerExclusive;
  if (!Number.isInteger(start) || !Number.isInteger(end) || start < 0 || end < start || end > manifest.blockCount) {
    throw new Error(`Invalid HIP layer segment: ${start}..${end}`);
  }
  if (!acceleration.hipResidentWeightCacheEnabled(session)) {
    return undefined;
  }
  if (!(await kernels.checkHipSupport()).available || !hipSegmentSupport(session, manifest, start, end).supported) {
    return undefined;
  }
  const epsilon = options.epsilon !== undefined ? options.epsilon : session.epsilon;
  const owned = [];
  const upload = (array) => {
    const ptr = kernels.deviceAlloc(array.byteLength);
    owned.push(ptr);
    kernels.copyToDevice(ptr, array);
    return ptr;
  };
  try {
    let freqFactors; // rope_freqs.weight (full-attention layers), one device copy
    const layers = [];
    for (let layer = start; layer < end; layer += 1) {
      const handle = async (name) => {
        const tensorName = `blk.${layer}.${name}.weight`;
        const tensor = session.getTensor(tensorName);
        const h = await acceleration.readHipWeightHandle(session, tensorName, tensor.type, tensor.dimensions[0],
          tensor.dimensions[1]);
        if (!h) {
          throw new Error(`declined: ${tensorName}`);
        }
        return h.handle;
      };
      const descriptor = {
        attnQ: await handle("attn_q"),
        attnK: await handle("attn_k"),
        attnV: valueShared(manifest, layer) ? 0n : await handle("attn_v"),
        attnOutput: await handle("attn_output"),
        ffnGate: await handle("ffn_gate"),
        ffnUp: await handle("ffn_up"),
        ffnDown: await handle("ffn_down"),
      };
      for (const [key, name] of Object.entries(NORMS)) {
        descriptor[key] = upload(await session.readF32Tensor(`blk.${layer}.${name}.weight`));
      }
      const scale = await session.readF32Tensor(`blk.${layer}.layer_output_scale.weight`);
      descriptor.layerOutputScale = scale[0] === undefined ? 1 : scale[0];
      const kind = layerKind(manifest, layer);
      let factors = 0n;
      if (kind !== "sliding-attention") {
        const tensor = tensorInfo(session, "rope_freqs.weight");
        if (tensor && tensor.type === "F32") {
          if (freqFactors === undefined) {
            freqFactors = upload(await session.readF32Tensor("rope_freqs.weight"));
          }
          factors = freqFactors;
        }
      }
      descriptor.attention = {
        headCount: manifest.headCount,
        headCountKv: (manifest.layerHeadCountKv && manifest.layerHeadCountKv[layer]) || manifest.headCountKv,
        headDim: HEAD_DIM,
        ropeDims: kind === "sliding-attention" ? manifest.rope.slidingDimensionCount : manifest.rope.fullDimensionCount,
        ropeFreqBase: kind === "sliding-attention" ? manifest.rope.slidingFreqBase : manifest.rope.fullFreqBase,
        ropeFreqFactors: factors,
        capacity: 0, // per state
        slidingWindow: kind === "sliding-attention" ? manifest.slidingWindow : 0,
        epsilon,
      };
      let ple;
      if (manifest.perLayerEmbeddingLength > 0) {
        ple = {
          inpGate: await handle("inp_gate"),
          proj: await handle("proj"),
          postNorm: upload(await session.readF32Tensor(`blk.${layer}.post_norm.weight`)),
        };
      }
      layers.push({ layer, headCountKv: descriptor.attention.headCountKv, descriptor, ple });
    }
    return new HipSegmentRunner({ session, manifest, epsilon, segmentStartLayer: start, segmentEndLayerExclusive: end },
      layers, owned, kernels);
  } catch (error) {
    for (const ptr of owned) {
      kernels.deviceFree(ptr);
    }
    if (error instanceof Error && error.message.startsWith("declined: ")) {
      return undefined;
    }
    throw error;
  }
}

module.exports = { HipSegmentRunner, createHipSegmentRunner, deviceRingFromHost, f16Bits, hipSegmentSupport };
