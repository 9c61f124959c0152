"""The Node N-API binding (heliopause_amd/napi): hp_hip.node + hip-kernels.js.

CPU: the addon loads in Node, exports the runner API of wasm-kernels.ts
(createWasmQuantizedWeightHandle 520-574 ... matMulQuantizedWasmResidentMulti
648-749) under its Hip names, and keeps that module's undefined-vs-throw
behaviour and messages.  GPU: projections, gate/up + GeGLU and head + top-k
issued from Node (async, on the libuv pool) match the oracle bit for bit.
GGUF: ggufOpen/ggufInfo from Node against the oracle's parseGguf (CPU), and
HipGgufWeights loading a file and projecting with it (GPU).
"""
import json
import math
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from heliopause_amd import synthetic as S

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "tests" / "napi_driver.js"
ADDON = ROOT / "heliopause_amd" / "napi" / "hp_hip.node"
NODE = shutil.which("node")

needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _node(*args, timeout=90):
    if not ADDON.exists():
        pytest.fail(f"{ADDON} is not built (run __graft_entry__.build())")
    r = subprocess.run([NODE, str(DRIVER), *args], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


@needs_node
def test_addon_api_without_gpu():
    out = _node("api")
    assert out["exports"] == sorted([
        "HipGgufFile", "HipGgufWeights", "openHipGgufFile", "DEFAULT_SAMPLING_SEED", "createHipSamplingState",
        "matMulQuantizedHipResidentTopKSample", "resolveGenerationSamplingOptions",
        "assertHipOk", "checkHipSupport", "createHipQuantizedWeightHandle", "hipResidentWeightStats",
        "matMulGegluHipResident", "matMulQuantizedHipResident", "matMulQuantizedHipResidentMulti",
        "matMulQuantizedHipResidentTopK", "quantizedTypeId", "releaseHipQuantizedWeightHandle",
        "copyToDevice", "copyToHost", "deviceAlloc", "deviceFree", "headTopKDevice", "runDecodeLayers"])
    assert set(out["support"]) >= {"available"}
    assert out["typeIds"] == [1, 2, 3, 4, 5, 6, 0]                  # wasm-kernels.ts:1908-1923
    assert out["unknownType"] == "undefined"
    assert out["zeroShape"] == "Resident quantized weight shape mismatch: inputSize=0 rowCount=1"
    assert out["scaleShape"] == "Q6_K scale shape mismatch: 100"   # wasm-kernels.ts:1935-1937
    assert out["multiOne"] == "undefined" and out["multiFive"] == "undefined"
    assert out["handleShape"] == "Resident quantized matmul handle shape mismatch: 256x1"
    assert out["inputShape"] == "Resident quantized matmul input shape mismatch: 255"
    assert out["releasedHandle"] == "Resident quantized matmul instance 1 is not available"
    assert out["multiShape"] == "Resident quantized multi matmul handle shape mismatch: 512"
    assert out["assertShape"] == "k hip shape mismatch"
    assert out["assertType"] == "k hip unsupported type"
    assert out["sampling"] == {"doSample": True, "temperature": 1, "topP": 0.95, "topK": 64, "seed": 0x48454C49,
                               "logitsTopK": 64}                      # generation.test.ts:12-30
    assert out["samplingGreedy"] == 1 and out["samplingTopK"] == 64
    assert out["samplingBadTemp"].startswith("temperature") and out["samplingBadTopP"].startswith("topP")
    assert out["samplingState"] == [0xFFFFFFFF]


@needs_node
@pytest.mark.gpu
def test_addon_projections_bit_exact(oracle, tmp_path):
    k, m, top_k, softcap = 2560, 2, 40, 30.0
    seed = S.derive(S.BASE_SEED, "napi")
    specs = [("Q4_K", 64), ("Q6_K", 48), ("Q4_K", 33), ("Q4_K", 96), ("Q4_K", 96), ("Q6_K", 3000)]
    ws = [S.weight_blocks(t, S.derive(seed, i), r, k) for i, (t, r) in enumerate(specs)]
    x = S.activations(seed, m, k)
    for i, w in enumerate(ws):
        (tmp_path / f"w{i}.bin").write_bytes(np.ascontiguousarray(w).tobytes())
    (tmp_path / "x.bin").write_bytes(x.astype(np.float32).tobytes())
    spec = {"inputSize": k, "columns": m, "topK": top_k, "softcap": softcap, "seed": 4242,
            "weights": [{"type": t, "rows": r, "file": f"w{i}.bin"} for i, (t, r) in enumerate(specs)]}
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print(f"napi k={k} m={m}", flush=True)
    res = _node("run", str(tmp_path))

    tid = {"Q4_K": 1, "Q6_K": 3}
    refs = [oracle.matmul(tid[t], w, x, r) for (t, r), w in zip(specs, ws)]

    def same(name, ref):
        got = np.fromfile(tmp_path / name, dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(ref, np.float32).reshape(-1).view(np.uint32)), name

    same("out_single.bin", refs[0])
    for i in range(3):
        same(f"out_multi{i}.bin", refs[i])
    same("out_geglu.bin", oracle.geglu(refs[3].reshape(-1), refs[4].reshape(-1)))
    top = json.loads((tmp_path / "out_topk.json").read_text())
    for col in range(m):
        capped = np.array([oracle.softcap(float(v), softcap) for v in refs[5].reshape(m, -1)[col]], np.float32)
        ids, vals = oracle.topk(capped, top_k)
        assert [c["id"] for c in top[col]] == ids.tolist()
        got_vals = np.array([c["value"] for c in top[col]], np.float32)
        assert np.array_equal(got_vals.view(np.uint32), vals.view(np.uint32))
    assert res["residentBefore"] > 0 and res["residentAfter"] == 0 and res["handlesAfter"] == 0
    assert res["mismatch"] == "Resident quantized matmul handle shape mismatch: 2560x64"
    from oracle import sampling as SM

    sampled = json.loads((tmp_path / "out_sample.json").read_text())
    opts = SM.resolve_options(temperature=0.8, topP=0.9, topK=40, seed=4242)
    rng = SM.DeterministicRng(4242)
    for call in sampled["sampled"]:
        for col in range(m):
            capped = np.array([oracle.softcap(float(v), softcap) for v in refs[5].reshape(m, -1)[col]], np.float32)
            ids, vals = oracle.topk(capped, 40)
            cands = [{"id": int(i), "value": float(v)} for i, v in zip(ids, vals)]
            dist = SM.token_sampling_distribution(cands, opts)
            assert call[col]["token"] == SM.sample_next_token(cands, opts, rng)
            assert [d["probability"] for d in call[col]["distribution"]] == [d["probability"] for d in dist]
    assert sampled["state"] == rng.state


def _jsonable(v):
    """The oracle's parse as the driver serialises it: big integers (offsets,
    data start) as strings, non-finite floats as JSON null."""
    if isinstance(v, dict):
        return {k: _jsonable(x) for k, x in v.items()}
    if isinstance(v, list):
        return [_jsonable(x) for x in v]
    if isinstance(v, float) and not math.isfinite(v):
        return None
    return v


@needs_node
@pytest.mark.parametrize("seed", [3, 5, 8, 13, 21])
def test_addon_gguf_parse_matches_oracle(tmp_path, seed):
    """ggufOpen / ggufInfo from Node against the oracle's parseGguf."""
    from oracle import gguf as OG
    from test_gguf import random_file

    data, *_ = random_file(seed)
    path = tmp_path / "f.gguf"
    path.write_bytes(data)
    for max_sample, keys in ((16, ()), (1, ("key.0", "key.1"))):
        got = _node("gguf", str(path), str(max_sample), *keys)
        ref = OG.parse_gguf(data, max_sample, keys)
        for t, r in zip(got["tensors"], ref["tensors"]):
            assert t.pop("byteLength", None) == (OG.tensor_byte_length(r) if r["type"] in OG.GGML_TYPE_STORAGE else None)
            r["offset"], r["dataOffset"] = str(r["offset"]), str(r["dataOffset"])
        ref["dataStart"] = str(ref["dataStart"])
        for k in ("alignment", "fileSize"):
            got.pop(k)
        assert got == _jsonable(ref)


@needs_node
@pytest.mark.gpu
def test_addon_gguf_upload_bit_exact(oracle, tmp_path):
    """A GGUF file loaded from Node (HipGgufWeights over ggufUpload) gives
    projections bit-exact with the oracle on the file's tensor bytes."""
    from heliopause_amd import gguf as G

    k, m = 2560, 2
    specs = [("blk.0.attn_q.weight", "Q4_K", 640), ("blk.0.attn_v.weight", "Q6_K", 512),
             ("blk.0.attn_norm.weight", "F32", 1), ("output.weight", "Q6_K", 9000)]
    tensors, ws = [], {}
    for i, (name, typ, rows) in enumerate(specs):
        if typ == "F32":
            data = S.random_bytes(S.derive(S.BASE_SEED, "napi-gguf", i), 4 * k)
        else:
            data = S.weight_blocks(typ, S.derive(S.BASE_SEED, "napi-gguf", i), rows, k)
            ws[name] = (typ, rows, data)
        tensors.append((name, [k, rows], G.GGML_TYPE_IDS[typ], data))
    G.write_gguf(tmp_path / "model.gguf", [("general.architecture", G.GGUF_STRING, "gemma4")], tensors)
    x = S.activations(S.derive(S.BASE_SEED, "napi-gguf-x"), m, k)
    (tmp_path / "x.bin").write_bytes(x.astype(np.float32).tobytes())
    (tmp_path / "case.json").write_text(json.dumps({"columns": m}))
    print("napi gguf upload", flush=True)
    res = _node("ggufrun", str(tmp_path))
    assert res["unsupported"] == ["blk.0.attn_norm.weight"] and res["sameHandle"]
    assert res["handlesAfter"] == 0 and res["bytes"] == sum(w[2].size for w in ws.values())
    for name, (typ, rows, data) in ws.items():
        got = np.fromfile(tmp_path / f"out_{name}.bin", dtype=np.float32)
        ref = oracle.matmul({"Q4_K": 1, "Q6_K": 3}[typ], data, x, rows)
        assert np.array_equal(got.view(np.uint32), ref.reshape(-1).view(np.uint32)), name
