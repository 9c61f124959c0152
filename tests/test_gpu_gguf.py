"""GGUF file -> HBM-resident handles (hp_hip_weight_upload_gguf) on the GPU.

The handles uploaded straight from a file must behave exactly like handles
uploaded from the same bytes in memory: projections bit-exact with the
oracle on the tensor bytes, dequantised rows bit-exact, unsupported block
types reported for fallback, and a failed load leaving no handle behind.
"""
import numpy as np
import pytest

from heliopause_amd import gguf as G
from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu

K = 2560


def _model_file(path, specs):
    tensors = []
    for i, (name, typ, k, rows) in enumerate(specs):
        if typ in ("Q4_K", "Q6_K"):
            data = S.weight_blocks(typ, S.derive(S.BASE_SEED, "gguf", i), rows, k)
        else:
            nbytes = {"F32": 4 * k * rows, "Q8_0": k // 32 * 34 * rows}[typ]
            data = S.random_bytes(S.derive(S.BASE_SEED, "gguf-other", i), nbytes)
        tensors.append((name, [k, rows], G.GGML_TYPE_IDS[typ], data))
    md = [("general.architecture", G.GGUF_STRING, "gemma4"), ("general.alignment", G.GGUF_UINT32, 64)]
    G.write_gguf(path, md, tensors, alignment=64)
    return {name: data for name, _, _, data in tensors}


def test_upload_from_file_matches_oracle(hip, oracle, tmp_path):
    specs = [("blk.0.attn_q.weight", "Q4_K", K, 2048), ("blk.0.attn_k.weight", "Q4_K", K, 512),
             ("blk.0.attn_v.weight", "Q6_K", K, 512), ("blk.0.ffn_down.weight", "Q4_K", 10240, 300),
             ("blk.0.attn_norm.weight", "F32", 256, 1), ("token_embd_q8.weight", "Q8_0", K, 64),
             ("output.weight", "Q6_K", K, 20000)]          # 42 MB: many 8 MiB chunks over all readers
    path = tmp_path / "model.gguf"
    data = _model_file(path, specs)
    print(f"gguf upload {path.stat().st_size} bytes", flush=True)
    before = hip.hipResidentWeightStats()["handleCount"]
    with G.GgufFile(path) as f:
        w = G.GgufHipWeights(f)
        handles = w.upload_all()
        assert handles["blk.0.attn_norm.weight"] is None and handles["token_embd_q8.weight"] is None
        assert w.handle("blk.0.attn_q.weight") is handles["blk.0.attn_q.weight"] and w.hits == 1
        x = S.activations(S.derive(S.BASE_SEED, "gguf-x"), 2, K)
        for name, typ, k, rows in specs:
            h = handles[name]
            if h is None:
                continue
            xin = x if k == K else S.activations(S.derive(S.BASE_SEED, "gguf-x", k), 2, k)
            got = hip.matMulQuantizedHipResident(h, xin, k, rows, 2)
            ref = oracle.matmul({"Q4_K": 1, "Q6_K": 3}[typ], data[name], xin, rows, threads=8)
            assert np.array_equal(got.view(np.uint32), ref.reshape(-1).view(np.uint32)), name
            tid = {"Q4_K": 1, "Q6_K": 3}[typ]
            probe = min(rows, 7)
            deq = hip.dequantizeHipResident(h, rows - probe, probe)
            tail = np.ascontiguousarray(data[name]).reshape(rows, -1)[rows - probe:]
            ref_rows = oracle.dequantize(tid, tail.reshape(-1), probe * k).reshape(probe, k)
            assert np.array_equal(deq.view(np.uint32), ref_rows.view(np.uint32)), name
        assert hip.hipResidentWeightStats()["handleCount"] == before + 5
        w.release()
    assert hip.hipResidentWeightStats()["handleCount"] == before


def test_failed_load_leaves_nothing(hip, tmp_path):
    """A tensor whose data runs past the end of the file fails the whole call
    (HP_ERR_IO) and no handle of that call survives; a 3-D Q4_K tensor is a
    shape error."""
    path = tmp_path / "cut.gguf"
    _model_file(path, [("a", "Q4_K", K, 64), ("b", "Q6_K", K, 64)])
    raw = path.read_bytes()
    path.write_bytes(raw[:-1000])
    before = hip.hipResidentWeightStats()["handleCount"]
    with G.GgufFile(path) as f:
        with pytest.raises(RuntimeError, match="past the end of the file"):
            G.GgufHipWeights(f).upload_all()
    assert hip.hipResidentWeightStats()["handleCount"] == before
    blocks = S.weight_blocks("Q4_K", 5, 4, K)
    G.write_gguf(tmp_path / "cube.gguf", [], [("c", [K, 2, 2], G.GGML_TYPE_IDS["Q4_K"], blocks)])
    with G.GgufFile(tmp_path / "cube.gguf") as f:
        with pytest.raises(ValueError, match="shape mismatch"):
            G.GgufHipWeights(f).upload_all()
    assert hip.hipResidentWeightStats()["handleCount"] == before
