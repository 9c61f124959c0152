"""Pins the oracle's decoder-layer steps (CPU only).

- rmsNormVector / rmsNormRowsNoWeight (layers.ts:834-885): closed forms
  (constant and one-element rows, zero rows), exact invariance under
  power-of-two scaling, unit mean square, and f64 agreement.
- ropeNeox (layers.ts:990-1033): the angles, pow and trigonometry against
  the JS engine's own values (tests/golden/v8_rope.json, written by
  tests/golden/make_v8_rope.js under this container's Node): unit pairs must
  come out as f32(cos) / f32(sin) of the engine's angles; identity at
  position 0, untouched dimensions beyond nDims, pair norms preserved.
- hp_gqa_attention_f32 (lib.rs:538-654): status codes, one key returns its
  value exactly, identical keys give the value mean, ring wrap equals the
  compacted cache, the GQA head mapping, and agreement with an f64 softmax
  attention.
- castF16Rows: numpy's round-to-nearest-even f16 with the reference's
  saturation at 65504.
- forward_layer: with zero O and down weights the layer reduces to the
  residual stream times the layer scale, and the cache slot holds the f16
  of the rotated, normed key.
"""
import base64
import json
import math
from pathlib import Path

import numpy as np
import pytest

from heliopause_amd import synthetic as S

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def D(oracle):
    from oracle import decode_layer

    return decode_layer


def test_rms_norm_closed_forms(D):
    w = np.ones(7, np.float32)
    out = D.rms_norm_rows(np.full(7, 3.0, np.float32), w, 0.0)
    assert np.all(out == 1.0)                                   # c / sqrt(c^2) == 1 exactly for c = 3
    one = D.rms_norm_rows(np.array([2.5], np.float32), np.array([0.5], np.float32), 1e-6)
    assert one[0] == np.float32((2.5 * (1.0 / math.sqrt(6.25 + 1e-6))) * 0.5)
    assert np.all(D.rms_norm_rows(np.zeros(64, np.float32), np.ones(64, np.float32), 1e-6) == 0.0)
    nw = D.rms_norm_rows(np.array([3.0, 4.0], np.float32), None, 0.0)
    assert np.array_equal(nw, np.array([3 / math.sqrt(12.5), 4 / math.sqrt(12.5)], np.float32))


def test_rms_norm_invariants(D):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 2560)).astype(np.float32)
    w = np.ones(2560, np.float32)
    base = D.rms_norm_rows(x, w, 0.0)
    for k in (-6, 3, 20):                                       # sums of squares scale by 4^k exactly
        assert np.array_equal(D.rms_norm_rows(x * np.float32(2.0 ** k), w, 0.0), base)
    assert np.allclose(np.mean(base.astype(np.float64) ** 2, axis=1), 1.0, rtol=1e-6)
    x64 = x.astype(np.float64)
    wr = rng.standard_normal(2560).astype(np.float32)
    ref = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-6) * wr
    got = D.rms_norm_rows(x, wr, 1e-6)
    assert np.max(np.abs(got - ref)) <= 2.0 ** -22 * np.max(np.abs(ref))


def _golden_cases():
    data = json.loads((GOLDEN / "v8_rope.json").read_text())
    for c in data["cases"]:
        dec = lambda k: np.frombuffer(base64.b64decode(c[k]), "<f8")  # noqa: E731
        yield c, dec("theta_f64le_base64"), dec("cos_f64le_base64"), dec("sin_f64le_base64")


def test_rope_matches_engine_angles(D):
    count = 0
    for c, theta, cos, sin in _golden_cases():
        n = c["nDims"]
        half = n // 2
        # head 0: unit x0 (-> cos, sin); head 1: unit x1 (-> -sin, cos)
        x = np.zeros((2, 256), np.float32)
        x[0, :half] = 1.0
        x[1, half:n] = 1.0
        out = D.rope_neox(x, [c["position"]], n, float(c["base"]))
        f = lambda a: a.astype(np.float32)  # noqa: E731
        assert np.array_equal(out[0, :half], f(cos)), (c["base"], n, c["position"])
        assert np.array_equal(out[0, half:n], f(sin))
        assert np.array_equal(out[1, :half], f(-sin))
        assert np.array_equal(out[1, half:n], f(cos))
        assert np.array_equal(D.rope_theta_table(c["position"], n, float(c["base"])), theta)
        count += half
    assert count == 4224


def test_rope_identity_norms_and_tail(D):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 256)).astype(np.float32)
    assert np.array_equal(D.rope_neox(x, [0], 256, 10000.0), x)
    out = D.rope_neox(x, [4096], 128, 10000.0)
    assert np.array_equal(out[:, 128:], x[:, 128:])              # dims beyond nDims pass through
    a = np.hypot(x[:, :64].astype(np.float64), x[:, 64:128])
    b = np.hypot(out[:, :64].astype(np.float64), out[:, 64:128])
    assert np.allclose(a, b, rtol=1e-6, atol=1e-6)
    ff = np.full(64, 2.0, np.float32)                            # theta / 2 at every pair
    assert np.array_equal(D.rope_neox(x, [8], 128, 10000.0, ff)[:, 0], D.rope_neox(x, [4], 128, 10000.0)[:, 0])


def test_cast_f16_rows(D):
    rng = np.random.default_rng(5)
    v = (rng.standard_normal(100000) * 50).astype(np.float32)
    assert np.array_equal(D.cast_f16_rows(v), v.astype(np.float16).astype(np.float32))
    big = np.array([65504.0, 65519.0, 65520.0, 1e9, -7e4], np.float32)
    assert np.array_equal(D.cast_f16_rows(big), np.array([65504, 65504, 65504, 65504, -65504], np.float32))


def _attn(D, q, keys, values, count, start, cap, nq, nkv, mask=None):
    return D.gqa_attention_f32(q, keys, values, head_size=256, query_heads=nq, kv_heads=nkv, token_count=1,
                               kv_count=count, kv_start=start, capacity=cap, mask=mask)


def test_attention_status_codes(D):
    q = np.zeros(256, np.float32)
    kv = np.zeros(4 * 256, np.float32)
    assert _attn(D, q, kv, kv, 2, 0, 4, 1, 1)[0] == 0
    assert _attn(D, q, kv[:-1], kv, 2, 0, 4, 1, 1)[0] == 1      # key length
    assert _attn(D, q, kv, kv, 5, 0, 4, 1, 1)[0] == 2           # more tokens than capacity
    assert _attn(D, np.zeros(3 * 256, np.float32), np.zeros(4 * 2 * 256, np.float32),
                 np.zeros(4 * 2 * 256, np.float32), 2, 0, 4, 3, 2)[0] == 2  # 3 % 2 != 0


def test_attention_closed_forms(D):
    rng = np.random.default_rng(6)
    cap = 16
    q = rng.standard_normal(256).astype(np.float32)
    keys = rng.standard_normal((cap, 1, 256)).astype(np.float32)
    values = rng.standard_normal((256, 1, cap)).astype(np.float32)     # dim-head-token
    rc, out = _attn(D, q, keys, values, 1, 5, cap, 1, 1)
    assert rc == 0 and np.array_equal(out, values[:, 0, 5])            # one key: its value
    same = np.repeat(keys[:1], cap, axis=0)
    rc, out = _attn(D, q, same, values, cap, 0, cap, 1, 1)
    assert np.allclose(out, values[:, 0, :].astype(np.float64).mean(axis=1), rtol=1e-5, atol=1e-6)


def test_attention_ring_wrap_equals_compacted(D):
    rng = np.random.default_rng(7)
    cap, count, start, nq, nkv = 40, 30, 25, 4, 2
    q = rng.standard_normal(nq * 256).astype(np.float32)
    keys = rng.standard_normal((cap, nkv, 256)).astype(np.float32)
    values = rng.standard_normal((256, nkv, cap)).astype(np.float32)
    slots = (start + np.arange(count)) % cap
    rc1, ring = _attn(D, q, keys, values, count, start, cap, nq, nkv)
    rc2, comp = _attn(D, q, np.ascontiguousarray(keys[slots]), np.ascontiguousarray(values[:, :, slots]), count, 0,
                      count, nq, nkv)
    assert rc1 == rc2 == 0 and np.array_equal(ring, comp)
    # GQA: swapping the kv heads swaps the outputs of the two query groups
    rc3, sw = _attn(D, np.concatenate([q[512:], q[:512]]), np.ascontiguousarray(keys[:, ::-1]),
                    np.ascontiguousarray(values[:, ::-1]), count, start, cap, nq, nkv)
    assert rc3 == 0 and np.array_equal(sw, np.concatenate([ring[512:], ring[:512]]))


def test_attention_near_f64_softmax(D):
    rng = np.random.default_rng(8)
    cap, nq, nkv = 300, 8, 2
    q = rng.standard_normal((nq, 256)).astype(np.float32) * 0.1
    keys = rng.standard_normal((cap, nkv, 256)).astype(np.float16).astype(np.float32)
    values = rng.standard_normal((256, nkv, cap)).astype(np.float16).astype(np.float32)
    rc, out = _attn(D, q, keys, values, cap, 0, cap, nq, nkv)
    assert rc == 0
    out = out.reshape(nq, 256)
    for h in range(nq):
        g = h // (nq // nkv)
        qh = q[h].astype(np.float16).astype(np.float64)
        s = keys[:, g, :].astype(np.float64) @ qh
        p = np.exp(s - s.max())
        ref = (values[:, g, :].astype(np.float64) @ p) / p.sum()
        assert np.max(np.abs(out[h] - ref)) <= 2e-5 * max(1.0, np.max(np.abs(ref))), h


def test_forward_layer_residual_path(D, oracle):
    """Zero O and down weights: o = 0 and y = 0 normalise to 0, so the
    output is the input times the layer scale; the cache slot holds
    f16(rope(norm(k)))."""
    hidden, nq, nkv, ffn, cap = 512, 2, 1, 256, 8
    rng = np.random.default_rng(9)
    seed = S.derive(S.BASE_SEED, "oracle-layer")

    def zero_blocks(t, rows, k):
        return np.zeros((rows, oracle.row_bytes(t, k)), np.uint8)

    w = {
        "attn_q": (1, S.q4_k_blocks(S.derive(seed, "q"), nq * 256, hidden), nq * 256),
        "attn_k": (1, S.q4_k_blocks(S.derive(seed, "k"), nkv * 256, hidden), nkv * 256),
        "attn_v": (3, S.q6_k_blocks(S.derive(seed, "v"), nkv * 256, hidden), nkv * 256),
        "attn_output": (1, zero_blocks(1, hidden, nq * 256), hidden),
        "ffn_gate": (1, S.q4_k_blocks(S.derive(seed, "g"), ffn, hidden), ffn),
        "ffn_up": (1, S.q4_k_blocks(S.derive(seed, "u"), ffn, hidden), ffn),
        "ffn_down": (3, zero_blocks(3, hidden, ffn), hidden),
    }
    norms = {n: (1.0 + 0.1 * rng.standard_normal(hidden if n not in ("attn_q_norm", "attn_k_norm") else 256))
             .astype(np.float32) for n in ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm",
                                           "ffn_norm", "post_ffw_norm")}
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    layer = D.Layer(weights=w, norms=norms, key_cache=kc, value_cache=vc, head_count=nq, head_count_kv=nkv,
                    output_scale=0.75)
    x = rng.standard_normal(hidden).astype(np.float32)
    out = D.forward_layer(layer, x, 11)
    assert np.array_equal(out, (x * np.float32(0.75)).astype(np.float32))
    kn = D.rms_norm_rows(layer.trace["k"].reshape(nkv, 256), norms["attn_k_norm"], 1e-6)
    assert np.array_equal(kc[:, 11 % cap], D.rope_neox(kn, [11], 256, 10000.0).astype(np.float16))
    assert np.array_equal(vc[:, 11 % cap], D.rms_norm_rows(layer.trace["v"].reshape(nkv, 256), None, 1e-6)
                          .astype(np.float16))


def _ple_layer(D, oracle, eps=1e-6, P=256):
    """A small layer with the per-layer input step (hidden 512, P = 256)."""
    hidden, nq, nkv, ffn, cap = 512, 2, 1, 256, 8
    seed = S.derive(S.BASE_SEED, "oracle-ple")
    rng = np.random.default_rng(13)
    w = {
        "attn_q": (1, S.q4_k_blocks(S.derive(seed, "q"), nq * 256, hidden), nq * 256),
        "attn_k": (1, S.q4_k_blocks(S.derive(seed, "k"), nkv * 256, hidden), nkv * 256),
        "attn_v": (3, S.q6_k_blocks(S.derive(seed, "v"), nkv * 256, hidden), nkv * 256),
        "attn_output": (1, S.q4_k_blocks(S.derive(seed, "o"), hidden, nq * 256), hidden),
        "ffn_gate": (1, S.q4_k_blocks(S.derive(seed, "g"), ffn, hidden), ffn),
        "ffn_up": (1, S.q4_k_blocks(S.derive(seed, "u"), ffn, hidden), ffn),
        "ffn_down": (3, S.q6_k_blocks(S.derive(seed, "d"), hidden, ffn), hidden),
        "inp_gate": (1, S.q4_k_blocks(S.derive(seed, "ig"), P, hidden), P),
        "proj": (1, S.q4_k_blocks(S.derive(seed, "pr"), hidden, P), hidden),
    }
    norms = {n: (1.0 + 0.1 * rng.standard_normal(256 if n in ("attn_q_norm", "attn_k_norm") else hidden))
             .astype(np.float32) for n in ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm",
                                           "ffn_norm", "post_ffw_norm", "post_norm")}
    kc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)
    vc = rng.standard_normal((nkv, cap, 256)).astype(np.float16)

    def make():
        return D.Layer(weights=dict(w), norms=dict(norms), key_cache=kc.copy(), value_cache=vc.copy(),
                       head_count=nq, head_count_kv=nkv, epsilon=eps, output_scale=0.875)
    x = (rng.standard_normal((3, hidden)) * 4).astype(np.float32)
    pli = rng.standard_normal((3, P)).astype(np.float32)
    return make, x, pli, w, norms


def test_per_layer_input_zero_input_is_the_plain_layer(D, oracle):
    """A zero per-layer input makes mixed = 0, proj . 0 = 0 and its norm 0:
    the layer's output equals the layer without the step, bit for bit; a
    layer given no per-layer input skips the step."""
    make, x, pli, _, _ = _ple_layer(D, oracle)
    plain = D.forward_layer(make(), x, 5)
    assert np.array_equal(D.forward_layer(make(), x, 5, np.zeros_like(pli)), plain)
    with_input = D.forward_layer(make(), x, 5, pli)
    assert not np.array_equal(with_input, plain)


def test_per_layer_input_scale_invariance(D, oracle):
    """With epsilon 0, scaling the per-layer input by a power of two scales
    mixed, its Q8_K scales and proj's output exactly, and post_norm's rms
    normalisation cancels it: the same bits."""
    make, x, pli, _, _ = _ple_layer(D, oracle, eps=0.0)
    a = D.forward_layer(make(), x, 5, pli)
    b = D.forward_layer(make(), x, 5, pli * np.float32(4.0))
    c = D.forward_layer(make(), x, 5, pli * np.float32(0.25))
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_per_layer_input_against_f64_formula(D, oracle):
    """The step against its formula in f64 over the dequantized weights:
    x + rmsnorm(W_proj (gelu(W_gate x) * u)) * post_norm, with gelu the
    tanh approximation (the f16 roundings and Q8_K inputs of the reference
    are inside the bar).  A missing gelu, a transposed weight or the input
    applied to the wrong factor moves it by O(1)."""
    make, x, pli, w, norms = _ple_layer(D, oracle)
    L = make()
    out = D.forward_layer(L, x, 5, pli)
    x2 = L.trace["ffn_residual"].astype(np.float64)
    Wg = oracle.dequantize(1, w["inp_gate"][1], 256 * 512).reshape(256, 512).astype(np.float64)
    Wp = oracle.dequantize(1, w["proj"][1], 512 * 256).reshape(512, 256).astype(np.float64)
    g = x2 @ Wg.T
    gelu = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3)))
    p = (gelu * pli.astype(np.float64)) @ Wp.T
    pn = p / np.sqrt(np.mean(p * p, axis=1, keepdims=True) + 1e-6) * norms["post_norm"]
    ref = (x2 + pn) * np.float64(np.float32(0.875))
    err = np.max(np.abs(out - ref)) / np.sqrt(np.mean(ref * ref))
    assert err < 2e-2, err
    # and the step's share is not negligible: without it the bar fails
    nople = x2 * np.float64(np.float32(0.875))
    assert np.max(np.abs(out - nople)) / np.sqrt(np.mean(ref * ref)) > 0.1
