"""The engine-side HIP runner (heliopause_amd/napi/hip/): projection dispatch
by tensor name with the engine's own path as the fallback, the session's
handle cache and the "hip" provider, driven from Node.

CPU: with a stand-in runner module and a mock ModelSession, the dispatch of
matMulWeight / matMulWeightBatch (wasm/layers.ts:559-716) -- HIP for Q4_K and
Q6_K, the fallback for every other type, for a disabled provider and for
options that switch the cache or batching off; undefined (fall back) versus
throw (shape mismatch) as wasm-kernels.ts behaves; the cache's shared
pending upload, hits, misses and shutdown (acceleration.ts:164-201, 93-112);
createHipProvider's runner (provider.ts:30-36, model-runner.ts:54-73).  On a
host without a GPU the real runner module answers undefined and the fallback
runs.
GPU: one decoder layer's projections by tensor name over a GGUF file (Q/K/V
batch, O, gate/up + GeGLU, gate/up batch, down, the head's top-40) match the
oracle bit for bit.

The device segment runner (napi/hip/segment-runner.js, SegmentRunner of
runner/segment-runner.ts:18-34): on the CPU with a stand-in device, which
segments it takes (and the reason for each it leaves to the WASM runner),
the layer descriptors it builds (per-kind RoPE parameters, the sliding
window, RoPE factors on full-attention layers only, the state's ring
capacities), the host caches copied into the device rings as f16, the rows
it returns (the model's last layer: the last token only), its errors, the
head call of runToken and that release frees every buffer; its f32 -> f16
conversion against numpy; shutdown while an upload is pending.  On the GPU:
two layers at the 42-layer model's shape (one sliding with a 1024-slot ring,
one full with RoPE factors) over a GGUF file, one decode token through
runTokensHidden against the oracle's layers, the next through runToken's
output norm, head and top-40, and the ms per token from Node.
"""
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from heliopause_amd import synthetic as S

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "tests" / "hip_runner_driver.js"
NODE = shutil.which("node")

needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _node(*args, timeout=120):
    r = subprocess.run([NODE, str(DRIVER), *args], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


@needs_node
def test_dispatch_fallback_and_errors():
    out = _node("dispatch")
    # Q4_K through the HIP handle; a concurrent second call shares the one upload
    assert out["single"] == [0, 1, 2, 3, 4, 5, 6, 7, 0, 1] and out["singleConcurrentSame"]
    assert out["reads"] == ["blk.0.attn_q.weight"]
    assert out["batch"] == [16, 8, 8]                         # Q/K/V as one multi call: [2 columns][rows]
    assert "multi 1,2,3" in out["log"]
    # the engine's path for what HIP does not take
    assert out["batchDeclined"] == "undefined"                # the engine's batch answered undefined
    assert out["q8"] == [-1, -1] and out["f32"] == [-1, -1]
    assert out["odd1"] == "undefined" and out["odd2"] == "undefined"
    assert out["fallbackCalls"] == ["blk.0.attn_q.weight+blk.0.odd.weight", "blk.0.q8.weight",
                                    "blk.0.attn_norm.weight", "blk.0.attn_q.weight"]
    # shape errors throw instead of falling back
    assert out["badHandle"] == "Resident quantized weight shape mismatch: inputSize=256 rowCount=13"
    assert out["badInput"] == "blk.0.attn_q.weight input shape mismatch: 300 is not a multiple of 256"
    assert out["noFallback"].startswith("HIP quantized matmul is unavailable for blk.0.q8.weight")
    assert out["batchOne"] == "undefined"
    assert out["geglu"] == 12 and "geglu 4,5" in out["log"]
    assert out["topk"] == [[{"id": 3, "value": 1.5}]] * 2 and "topk 6 k=40 softcap=30" in out["log"]
    # cache statistics (registered as the session's "hip" stats provider) and shutdown
    st = out["stats"]
    assert st["hipResidentWeightCacheEnabled"] and st["hipResidentWeightCacheCount"] == 6
    assert st["hipResidentWeightCacheBytes"] == 96 and st["hipResidentWeightCacheMisses"] == 7
    assert st["hipResidentWeightCacheHits"] >= 2
    assert out["afterShutdown"]["hipResidentWeightCacheCount"] == 0
    assert sorted(x for x in out["log"] if x.startswith("release")) == [f"release {i}" for i in range(1, 7)]
    # provider off / cache off / batching off
    assert out["offSingle"] == "undefined" and out["offFallback"] == [-1, -1]
    assert out["noCache"] == "undefined" and out["noBatch"] == "undefined"
    # the provider and its model runner
    p = out["provider"]
    assert p["name"] == "hip" and p["options"] == {"projectionBatching": True}
    assert p["runnerProvider"] == "hip" and p["graphNodes"] == {"marker": 1} and p["prepared"] == "prepared"
    assert p["segment"] == ["hip", 2, 5] and p["tokensHidden"] == 1 and p["tokenHidden"] == 2
    req = p["requirements"]
    assert req["provider"] == "hip" and req["canRunFullModel"] and not req["targetResourceConstrained"]
    assert req["gguf"] == "gguf" and req["manifest"] == "manifest" and req["contextLength"] == 4096
    assert req["memoryLimitBytes"] == 288 * 2**30
    assert out["missingEngine"] == "The HIP runner provider needs engine.createWasmModelRunner."


@needs_node
def test_runner_module_without_gpu_falls_back():
    """Only meaningful where no GPU is visible (this container): the real
    runner module reports the device missing and the engine's path runs."""
    out = _node("nogpu")
    if out["support"]["available"]:
        pytest.skip("a GPU is visible: the fall-back path is not taken here")
    assert out["out"] == [1, 2] and out["called"] == ["blk.0.attn_q.weight"]
    assert out["stats"]["hipResidentWeightCacheDeclined"] == 1


@needs_node
@pytest.mark.gpu
def test_layer_projections_by_name_bit_exact(oracle, tmp_path):
    """A synthetic layer of the 42-layer model (hidden 2560, FFN 10240) and a
    reduced head in a GGUF file; the projections are asked for by tensor
    name, as the engine's layers ask."""
    from heliopause_amd import gguf as G

    hidden, ffn, head_rows, m = 2560, 10240, 20000, 2
    specs = {"blk.0.attn_q.weight": ("Q4_K", 2048, hidden), "blk.0.attn_k.weight": ("Q4_K", 512, hidden),
             "blk.0.attn_v.weight": ("Q6_K", 512, hidden), "blk.0.attn_output.weight": ("Q4_K", hidden, 2048),
             "blk.0.ffn_gate.weight": ("Q4_K", ffn, hidden), "blk.0.ffn_up.weight": ("Q4_K", ffn, hidden),
             "blk.0.ffn_down.weight": ("Q6_K", hidden, ffn), "output.weight": ("Q6_K", head_rows, hidden)}
    seed = S.derive(S.BASE_SEED, "hip-runner-layer")
    ws, tensors = {}, []
    for i, (name, (typ, rows, k)) in enumerate(specs.items()):
        ws[name] = S.weight_blocks(typ, S.derive(seed, i), rows, k)
        tensors.append((name, [k, rows], G.GGML_TYPE_IDS[typ], ws[name]))
    tensors.append(("blk.0.attn_norm.weight", [hidden], G.GGML_TYPE_IDS["F32"],
                    np.ones(hidden, np.float32).view(np.uint8)))
    G.write_gguf(tmp_path / "model.gguf", [("general.architecture", G.GGUF_STRING, "gemma4")], tensors)
    xs = {"x_attn": hidden, "x_o": 2048, "x_ffn": hidden, "x_down": ffn, "x_head": hidden}
    inputs = {}
    for j, (name, k) in enumerate(xs.items()):
        inputs[name] = S.activations(S.derive(seed, "x", j), m, k)
        (tmp_path / f"{name}.bin").write_bytes(inputs[name].astype(np.float32).tobytes())
    (tmp_path / "case.json").write_text(json.dumps({"topK": 40, "softcap": 0}))
    print("hip runner layer by tensor name", flush=True)
    out = _node("layer", str(tmp_path), timeout=300)
    T = {"Q4_K": 1, "Q6_K": 3}

    def ref(name, x):
        typ, rows, _ = specs[name]
        return oracle.matmul(T[typ], ws[name], x, rows, threads=8).reshape(-1)

    def check(file, expect):
        got = np.fromfile(tmp_path / file, dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), expect.astype(np.float32).view(np.uint32)), file

    for i, name in enumerate(["blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.attn_v.weight"]):
        check(f"out_qkv{i}.bin", ref(name, inputs["x_attn"]))
    check("out_o.bin", ref("blk.0.attn_output.weight", inputs["x_o"]))
    gate, up = ref("blk.0.ffn_gate.weight", inputs["x_ffn"]), ref("blk.0.ffn_up.weight", inputs["x_ffn"])
    check("out_gateup0.bin", gate)
    check("out_gateup1.bin", up)
    check("out_ffn.bin", oracle.geglu(gate, up))
    check("out_down.bin", ref("blk.0.ffn_down.weight", inputs["x_down"]))
    logits = ref("output.weight", inputs["x_head"]).reshape(m, head_rows)
    for c in range(m):
        ids, vals = oracle.topk(logits[c], 40)
        assert [t["id"] for t in out["top"][c]] == ids.tolist()
        assert np.array_equal(np.array([t["value"] for t in out["top"][c]], np.float32).view(np.uint32),
                              vals.view(np.uint32))
    assert out["fallbackCalls"] == ["blk.0.attn_norm.weight"]
    assert out["stats"]["hipResidentWeightCacheCount"] == len(specs)
    assert sorted(out["reads"]) == sorted(specs)                    # each tensor read once


@needs_node
def test_segment_runner_on_a_stand_in_device():
    out = _node("segment")
    assert out["support"] == {"supported": True}
    assert out["supportPle"] == "blk.0.post_norm.weight"   # per-layer inputs need their step's tensors
    assert out["supportPleLength"] == "per-layer input length 100"
    assert out["supportKvShared"] == "layer 1 reads another layer's KV"
    assert out["supportWidth"] == "layer 1 head width 512/256"
    assert out["supportType"] == "blk.1.ffn_up.weight type Q8_0"
    assert out["supportHidden"] == "hidden size 4352"
    assert out["runnerProvider"] == ["hip", 0, 2]
    assert out["invalidSegment"] == "Invalid HIP layer segment: 1..3"
    assert out["fallbackProvider"] == ["hip", False]        # no inp_gate tensors: the relabelled WASM runner
    # the model's last layer: only the last token's row comes back
    assert out["lastOnly"] == [512, 2, 1, 300, 3, 1536]
    L0 = out["layer0"]
    assert [L0[k] for k in ("attnQ", "attnK", "attnV", "attnOutput", "ffnGate", "ffnUp", "ffnDown")] == \
        ["1", "2", "3", "4", "5", "6", "7"]
    assert L0["layerOutputScale"] == 0.5
    assert L0["attention"] == {"headCount": 4, "headCountKv": 2, "headDim": 256, "ropeDims": 128,
                               "ropeFreqBase": 10000, "ropeFreqFactors": "0", "capacity": 64,
                               "slidingWindow": 48, "epsilon": 1e-06}
    assert out["layer1Attention"] == {"headCount": 4, "headCountKv": 2, "headDim": 256, "ropeDims": 256,
                                      "ropeFreqBase": 1000000, "ropeFreqFactors": True, "capacity": 8192,
                                      "slidingWindow": 0, "epsilon": 1e-06}
    # host caches (key [slot][head][dim], value [dim][head][slot]) -> f16 [head][slot][dim]
    assert out["ringKey"][0] == out["ringKey"][1] and out["ringValue"][0] == out["ringValue"][1]
    assert out["freshRingZero"] and out["freshRows"] == [0, 1]
    assert out["norm0"] == pytest.approx([1.0, 1.001, 1.002])
    assert out["middleRows"] == [1536, 10, 2010]             # a middle segment: every row
    assert out["nonConsecutive"] == "The HIP segment runner takes consecutive positions."
    assert out["outside"] == "Position 8192 is outside context length 8192"
    assert out["notCausal"] == "The HIP segment runner runs causal attention only."
    assert out["badShape"] == "HIP segment input shape mismatch: 1536"
    rt = out["runToken"]
    assert rt["selected"] == 7 and rt["topK"] == 10 and rt["softcap"] == 30
    assert rt["readOutput"] and rt["outputNorm"] and rt["headInput"]
    assert out["middleRunToken"] == "runToken needs a segment that ends at the model's last layer."
    assert out["allocs"] == out["frees"] and out["leftBuffers"] == 0
    assert out["afterRelease"] == "The HIP segment runner was released."
    # per-layer inputs: the segment's layer (1) gets its own block of rows
    # ([layer][token][P]: layer 1 of 2 tokens starts at 512); a run without
    # them skips the step; a wrong length throws
    assert out["ple"] == {"hasGate": True, "postNorm": True, "first": 512.0, "last": 1023.0}
    assert out["pleSkipped"]
    assert out["pleShape"] == "Per-layer input shape mismatch: 10"


@needs_node
def test_f16_bits_match_numpy():
    """The runner's f32 -> f16 conversion (host caches into the device rings)
    against numpy's round-to-nearest-even, over normal, subnormal, tie,
    overflow, infinite and NaN inputs."""
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),             # f16 subnormals
        (rng.standard_normal(2000) * 1e-8).astype(np.float32),             # below the smallest
        np.array([65504, 65519.99, 65520, 1e6, -1e6, np.inf, -np.inf, 0.0, -0.0, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -25, 2.0 ** -14, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11], np.float32),
    ]).astype(np.float32)
    ties = (np.arange(-2048, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)  # halfway values
    vals = np.concatenate([vals, ties.astype(np.float32)])
    r = subprocess.run([NODE, str(DRIVER), "f16"], input=json.dumps(vals.view(np.uint32).tolist()),
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.array(json.loads(r.stdout), np.uint16)
    with np.errstate(over="ignore"):     # values past 65520 round to infinity, as they should
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    nan = subprocess.run([NODE, str(DRIVER), "f16"], input=json.dumps([0x7FC00000, 0xFFC00001]),
                         capture_output=True, text=True, timeout=60)
    assert json.loads(nan.stdout) == [0x7E00, 0xFE00]


@needs_node
def test_shutdown_during_upload_releases_the_late_handle():
    out = _node("race")
    assert out["got"] == "undefined"
    assert out["log"][0] == "release 99"                       # the late handle, released on arrival
    assert out["secondCall"] == "1"                             # a later call uploads afresh
    assert out["stats"]["hipResidentWeightCacheCount"] == 1


@needs_node
@pytest.mark.gpu
def test_segment_runner_two_layers_on_the_device(oracle, tmp_path):
    """Two layers at the 42-layer model's shape (hidden 2560, 8 query / 2 KV
    heads of 256, FFN 10240): layer 0 sliding (window 512, a 1024-slot ring,
    RoPE base 10^4), layer 1 full (a 4096-slot ring, RoPE base 10^6 with
    rope_freqs), both rings already holding positions (the state's host
    caches, f16-exact values, copied in).  One token through
    runTokensHidden at position 4000 against the oracle's two layers (the
    one-token layer bar, LAYER_TOL); the next token through runToken: top-40
    ids equal to the oracle's end to end (output norm and a 32768-row Q6_K
    head)."""
    from heliopause_amd import decode as DM
    from heliopause_amd import gguf as G
    from oracle import decode_layer as D

    LAYER_TOL = 3.5e-3
    shape = DM.ModelShape()
    hidden, nkv, head_rows, pos = shape.hidden, shape.head_count_kv, 32768, 4000
    caps, kinds = [1024, 4096], ["sliding-attention", "full-attention"]
    bases, window = [10000.0, 1000000.0], 512
    seed = S.derive(S.BASE_SEED, "hip-segment-runner")
    datas = [DM.layer_host_data(shape, seed, i, cache_fill=False) for i in range(2)]
    T = G.GGML_TYPE_IDS
    tensors = []
    for i, d in enumerate(datas):
        for name, (typ, blocks, rows, k) in d["weights"].items():
            tensors.append((f"blk.{i}.{name}.weight", [k, rows], T[typ], blocks))
        for name, w in d["norms"].items():
            tensors.append((f"blk.{i}.{name}.weight", [w.size], T["F32"], w.astype(np.float32).view(np.uint8)))
        tensors.append((f"blk.{i}.layer_output_scale.weight", [1], T["F32"],
                        np.array([d["output_scale"]], np.float32).view(np.uint8)))
    freqs = (1.0 + np.abs(S.normal(S.derive(seed, "freqs"), 128))).astype(np.float32)
    onorm = (1 + 0.1 * S.normal(S.derive(seed, "onorm"), hidden)).astype(np.float32)
    head = S.weight_blocks("Q6_K", S.derive(seed, "head"), head_rows, hidden)
    tensors += [("rope_freqs.weight", [128], T["F32"], freqs.view(np.uint8)),
                ("output_norm.weight", [hidden], T["F32"], onorm.view(np.uint8)),
                ("output.weight", [hidden, head_rows], T["Q6_K"], head)]
    G.write_gguf(tmp_path / "model.gguf", [("general.architecture", G.GGUF_STRING, "gemma4")], tensors)
    # the state's caches: f16-exact values in the host layout
    f16c = []
    for i, cap in enumerate(caps):
        kc = S.normal(S.derive(seed, "k", i), nkv * cap * 256).astype(np.float16).reshape(nkv, cap, 256)
        vc = S.normal(S.derive(seed, "v", i), nkv * cap * 256).astype(np.float16).reshape(nkv, cap, 256)
        f16c.append((kc, vc))
        (tmp_path / f"cache_{i}_key.bin").write_bytes(kc.astype(np.float32).transpose(1, 0, 2).tobytes())
        (tmp_path / f"cache_{i}_value.bin").write_bytes(vc.astype(np.float32).transpose(2, 0, 1).tobytes())
    x = (S.activations(S.derive(seed, "x"), 1, hidden) * 4).reshape(-1)
    x2 = (S.activations(S.derive(seed, "x2"), 1, hidden) * 4).reshape(-1)
    (tmp_path / "x.bin").write_bytes(x.astype(np.float32).tobytes())
    (tmp_path / "x2.bin").write_bytes(x2.astype(np.float32).tobytes())
    case = {"layers": 2, "hidden": hidden, "headCount": shape.head_count, "headCountKv": nkv, "kinds": kinds,
            "slidingWindow": window, "contextLength": 4096, "capacities": caps, "position": pos, "steps": 20,
            "topK": 40, "epsilon": shape.epsilon,
            "rope": {"slidingDimensionCount": 256, "fullDimensionCount": 256, "slidingFreqBase": bases[0],
                     "fullFreqBase": bases[1], "dimensionCount": 256, "dimensionSections": [], "freqBase": bases[0]}}
    (tmp_path / "case.json").write_text(json.dumps(case))
    print("segment runner on the device: 2 layers at the 42-layer shape", flush=True)
    out = _node("segment-gpu", str(tmp_path), timeout=600)
    assert out["provider"] == "hip"
    tid = {"Q4_K": 1, "Q6_K": 3}
    layers = []
    for i, d in enumerate(datas):
        layers.append(D.Layer(weights={n: (tid[t], b, r) for n, (t, b, r, _) in d["weights"].items()},
                              norms=dict(d["norms"]), key_cache=f16c[i][0].copy(), value_cache=f16c[i][1].copy(),
                              head_count=shape.head_count, head_count_kv=nkv, rope_dims=256,
                              rope_freq_base=bases[i], rope_freq_factors=None if i == 0 else freqs,
                              sliding_window=window if i == 0 else 0, epsilon=shape.epsilon,
                              output_scale=float(d["output_scale"])))
    h = x.copy()
    for L in layers:
        h = D.forward_layer(L, h, pos)
    got = np.fromfile(tmp_path / "out_hidden.bin", dtype=np.float32)
    err = float(np.max(np.abs(got.astype(np.float64) - h)) / np.sqrt(np.mean(h.astype(np.float64) ** 2)))
    print(f"runTokensHidden: err {err:.3e} of the row rms, identical {np.mean(got == h):.4f}", flush=True)
    assert err <= LAYER_TOL
    h2 = x2.copy()
    for L in layers:
        h2 = D.forward_layer(L, h2, pos + 1)
    normed = D.rms_norm_rows(h2[None], onorm, shape.epsilon)
    logits = oracle.matmul(3, head, normed, head_rows, threads=8)[0]
    ids, vals = oracle.topk(logits, 40)
    g_ids = [t["id"] for t in out["top"]]
    print(f"runToken: top-40 shared {len(set(g_ids) & set(ids.tolist()))}; "
          f"ms per token from Node: runTokensHidden {out['hiddenMs']:.3f}, runToken {out['tokenMs']:.3f} "
          f"(2 layers; runner set-up {out['createMs']} ms)", flush=True)
    assert g_ids == ids.tolist()
