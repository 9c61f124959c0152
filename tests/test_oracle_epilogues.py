"""Pins the oracle's tanh, gelu / GeGLU, softcap and topK (CPU only).

tanh is compared bit for bit with V8's Math.tanh outputs in
tests/golden/v8_tanh.json (written by tests/golden/make_v8_tanh.js).  gelu
(layers.ts:1062-1076) is checked at closed-form points and against an exact
f64 GELU of the f16-rounded input within one f16 step of the result.  topK
(runtime.ts:514-527) is checked against a brute-force lexicographic sort
(value descending, id ascending; -0 == +0; NaN after every number).
"""
import base64
import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_tanh_matches_v8(oracle):
    import ctypes

    L = oracle.lib()
    L.hpo_tanh.argtypes = [ctypes.c_double]
    L.hpo_tanh.restype = ctypes.c_double
    data = json.loads((GOLDEN / "v8_tanh.json").read_text())
    xs = np.frombuffer(base64.b64decode(data["x_f64le_base64"]), dtype="<f8")
    ys = np.frombuffer(base64.b64decode(data["tanh_f64le_base64"]), dtype="<f8")
    assert xs.size == data["count"] > 40000
    got = np.array([L.hpo_tanh(float(x)) for x in xs])
    bad = np.flatnonzero(got.view(np.uint64) != ys.view(np.uint64))
    assert bad.size == 0, (xs[bad[:3]], got[bad[:3]], ys[bad[:3]])


def test_gelu_closed_form_points(oracle):
    assert oracle.gelu(0.0) == 0.0
    assert math.copysign(1.0, oracle.gelu(-0.0)) == -1.0
    assert oracle.gelu(10.0) == 10.0 and oracle.gelu(12.5) == 12.5
    assert oracle.gelu(-10.0) == 0.0 and oracle.gelu(-50.0) == 0.0
    # 0.5 * (1 + tanh(sqrt(2/pi) * 1.044715)) = 0.84119..., nearest f16 0.84130859375
    assert oracle.gelu(1.0) == 0.84130859375


def test_gelu_near_exact_gelu(oracle):
    rng = np.random.default_rng(21)
    v = (rng.standard_normal(20000) * 4).astype(np.float32)
    v = v[np.abs(v) < 9.99]
    for x in v:
        xh = float(np.float16(x))
        exact = 0.5 * xh * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * xh * (1.0 + 0.044715 * xh * xh)))
        got = oracle.gelu(float(x))
        step = float(np.spacing(np.float16(abs(exact)))) if exact != 0 else 2.0 ** -24
        assert abs(got - exact) <= step + 1e-7 * abs(exact), (x, got, exact)


def test_geglu_is_rounded_product(oracle):
    rng = np.random.default_rng(22)
    g = (rng.standard_normal(4096) * 3).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    out = oracle.geglu(g, u)
    want = np.array([np.float32(np.float64(oracle.gelu(float(a))) * np.float64(b)) for a, b in zip(g, u)])
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def _brute_topk(v, k):
    keyed = sorted(range(len(v)), key=lambda i: (1 if np.isnan(v[i]) else 0, -(0.0 if np.isnan(v[i]) else v[i]), i))
    ids = np.array(keyed[:k], dtype=np.uint32)
    return ids, v[ids]


@pytest.mark.parametrize("n,k", [(1000, 40), (50, 40), (10, 40), (4096, 1), (300, 64), (5, 0)])
def test_topk_brute_force(oracle, n, k):
    rng = np.random.default_rng(n + k)
    v = rng.integers(-5, 6, n).astype(np.float32) * 0.5  # many ties
    v[rng.integers(0, n, max(1, n // 10))] = -0.0
    if n > 20:
        v[3] = np.nan
        v[17] = np.inf
    ids, vals = oracle.topk(v, k)
    ref_ids, ref_vals = _brute_topk(v, k)
    assert np.array_equal(ids, ref_ids)
    assert np.array_equal(vals.view(np.uint32), ref_vals.astype(np.float32).view(np.uint32))


def test_forward_graph_top2_order(oracle):
    """forward-graph.test.ts:281-316 expects ids [1, 0] with values
    [0.5715..., -0.1633...]: a lower value with a lower id ranks second."""
    logits = np.array([-0.16329389810562134, 0.5715285539627075, -0.9], dtype=np.float32)
    ids, vals = oracle.topk(logits, 2)
    assert list(ids) == [1, 0]
    assert np.allclose(vals, [0.5715285539627075, -0.16329389810562134], atol=2e-5)


def test_softcap(oracle):
    assert oracle.softcap(0.0, 30.0) == 0.0
    assert oracle.softcap(float("inf"), 30.0) == 30.0
    xs = np.linspace(-200, 200, 401)
    ys = [oracle.softcap(float(x), 30.0) for x in xs]
    assert all(a <= b for a, b in zip(ys, ys[1:]))
    assert all(abs(y) <= 30.0 for y in ys)
