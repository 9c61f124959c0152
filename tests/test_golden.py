"""Frozen vectors (tests/golden/fixtures.npz, written by make_fixtures.py):
the oracle must still reproduce them (CPU), and the HIP path must match
them bit for bit (GPU)."""
from pathlib import Path

import numpy as np
import pytest

FIX = Path(__file__).resolve().parent / "golden" / "fixtures.npz"


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_oracle_reproduces_fixtures(oracle, fx):
    assert _eq(oracle.matmul(1, fx["q4k_w"], fx["q4k_x"], 13), fx["q4k_out"])
    assert _eq(oracle.matmul(3, fx["q6k_w"], fx["q6k_x"], 7), fx["q6k_out"])
    qs, d, bs = oracle.quantize_q8_k(fx["q4k_x"])
    assert np.array_equal(qs, fx["q4k_x_qs"]) and _eq(d, fx["q4k_x_d"]) and np.array_equal(bs, fx["q4k_x_bsums"])
    outs = oracle.matmul_multi([1, 1, 3], [fx[f"multi_w{i}"] for i in range(3)], fx["multi_x"], [16, 8, 8])
    assert all(_eq(o, fx[f"multi_out{i}"]) for i, o in enumerate(outs))
    for r in range(2):
        ids, vals = oracle.topk(fx["topk_logits"][r], 40)
        assert np.array_equal(ids, fx["topk_ids"][r]) and _eq(vals, fx["topk_vals"][r])
    assert _eq(oracle.geglu(fx["geglu_gate"], fx["geglu_up"]), fx["geglu_out"])


@pytest.mark.gpu
def test_gpu_matches_fixtures(hip, fx):
    h = hip.createHipQuantizedWeightHandle("Q4_K", fx["q4k_w"], 512, 13)
    try:
        assert _eq(hip.matMulQuantizedHipResident(h, fx["q4k_x"], 512, 13, 3).reshape(3, 13), fx["q4k_out"])
        assert _eq(hip.dequantizeHipResident(h, 0, 13), fx["q4k_deq"])
    finally:
        hip.releaseHipQuantizedWeightHandle(h)
    qs, d, bs = hip.quantizeQ8KHip(fx["q4k_x"], 512, 3)
    assert np.array_equal(qs, fx["q4k_x_qs"]) and _eq(d, fx["q4k_x_d"]) and np.array_equal(bs, fx["q4k_x_bsums"])
    h = hip.createHipQuantizedWeightHandle("Q6_K", fx["q6k_w"], 2560, 7)
    try:
        assert _eq(hip.matMulQuantizedHipResident(h, fx["q6k_x"], 2560, 7, 2).reshape(2, 7), fx["q6k_out"])
        assert _eq(hip.dequantizeHipResident(h, 0, 2), fx["q6k_deq"])
    finally:
        hip.releaseHipQuantizedWeightHandle(h)
    hs = [hip.createHipQuantizedWeightHandle(t, fx[f"multi_w{i}"], 2560, r)
          for i, (t, r) in enumerate([("Q4_K", 16), ("Q4_K", 8), ("Q6_K", 8)])]
    try:
        outs = hip.matMulQuantizedHipResidentMulti(hs, fx["multi_x"], 2560, 4)
        assert all(_eq(o.reshape(4, -1), fx[f"multi_out{i}"]) for i, o in enumerate(outs))
    finally:
        for h in hs:
            hip.releaseHipQuantizedWeightHandle(h)
    got = hip.topKHip(fx["topk_logits"], 40)
    for r in range(2):
        assert [c["id"] for c in got[r]] == list(fx["topk_ids"][r])
        assert _eq([c["value"] for c in got[r]], fx["topk_vals"][r])
    assert _eq(hip.gegluHip(fx["geglu_gate"], fx["geglu_up"]), fx["geglu_out"])
