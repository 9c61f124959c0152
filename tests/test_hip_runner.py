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
