"""GPU parity: top-k over logits, the output head + top-k, and GeGLU.

Top-k bar: ids identical and values bit-identical to the oracle's restatement
of runtime.ts:514-527 (descending value, ties to the lower id, -0 == +0).
GeGLU bar: bit-identical to the oracle's restatement of layers.ts:450-456 and
1062-1076 (whose tanh is pinned to V8's Math.tanh).
"""
import numpy as np
import pytest

from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _check_rows(got, logits, k, oracle, softcap=0.0):
    for r, row in enumerate(np.atleast_2d(logits)):
        vals = row if softcap == 0.0 else np.array([oracle.softcap(float(v), softcap) for v in row], np.float32)
        ids, ref_vals = oracle.topk(vals, k)
        g_ids = np.array([c["id"] for c in got[r]], dtype=np.uint32)
        g_vals = np.array([c["value"] for c in got[r]], dtype=np.float32)
        assert np.array_equal(g_ids, ids), (r, g_ids[:8], ids[:8])
        assert np.array_equal(g_vals.view(np.uint32), ref_vals.view(np.uint32)), r


@pytest.mark.parametrize("rows,n,k", [(1, 262144, 40), (4, 262144, 40), (2, 100000, 64), (3, 4096, 1),
                                      (1, 10, 40), (2, 300000, 17), (1, 524288, 40)])
def test_topk_random(hip, oracle, rows, n, k):
    print(f"topk rows={rows} n={n} k={k}", flush=True)
    logits = S.activations(S.derive(S.BASE_SEED, "topk", rows, n), rows, n) * 4.0
    got = hip.topKHip(logits, k)
    _check_rows(got, logits, k, oracle)


def test_topk_ties_and_zero_signs(hip, oracle):
    n, k = 262144, 40
    rng = np.random.default_rng(5)
    logits = np.zeros((3, n), dtype=np.float32)
    logits[0] = rng.integers(-3, 4, size=n).astype(np.float32)      # massive ties
    logits[1, ::2] = -0.0                                              # -0 / +0 ties
    logits[1, 1000:1100] = 1.5
    logits[2] = rng.standard_normal(n).astype(np.float32)
    logits[2, 7] = np.nan                                              # NaN ranks last
    logits[2, 9] = np.inf
    logits[2, 11] = -np.inf
    logits[2, 262143] = logits[2].max()                                # tie at the top, high id
    got = hip.topKHip(logits, k)
    _check_rows(got, logits, k, oracle)
    nan_row = np.full((1, 50), np.nan, dtype=np.float32)
    nan_row[0, 3] = 1.0
    _check_rows(hip.topKHip(nan_row, 40), nan_row, 40, oracle)


@pytest.mark.parametrize("k", [40, 64])
def test_topk_adversarial_orders(hip, oracle, k):
    """Inputs that defeat the chunk-maximum filter (thousands of candidates):
    ascending and descending logits, all equal, almost all -inf, one hot
    cluster.  Exercises the radix-select path of the final step."""
    n = 262144
    rng = np.random.default_rng(k)
    base = rng.standard_normal(n).astype(np.float32)
    rows = np.stack([np.sort(base), np.sort(base)[::-1], np.full(n, 30.0, np.float32),
                     np.where(rng.random(n) < 1e-4, base, -np.inf).astype(np.float32), base.copy()])
    rows[4, 5000:5100] += 10.0
    print(f"topk adversarial k={k}", flush=True)
    _check_rows(hip.topKHip(rows, k), rows, k, oracle)


def test_topk_row_batches_and_reuse(hip, oracle):
    """More rows than one launch holds (batches of 16), then calls of other
    shapes reusing the same scratch: its counters must return to zero."""
    logits = S.activations(S.derive(S.BASE_SEED, "topk-batches"), 37, 5000) * 3.0
    print("topk rows=37 n=5000", flush=True)
    _check_rows(hip.topKHip(logits, 40), logits, 40, oracle)
    small = logits[:3, :1500].copy()
    _check_rows(hip.topKHip(small, 7), small, 7, oracle)
    _check_rows(hip.topKHip(logits, 40), logits, 40, oracle)


def test_topk_softcap(hip, oracle):
    logits = S.activations(S.derive(S.BASE_SEED, "softcap"), 2, 65536) * 20.0
    _check_rows(hip.topKHip(logits, 40, softcap=30.0), logits, 40, oracle, softcap=30.0)


@pytest.mark.parametrize("rows,m", [(20000, 1), (20000, 4)])
def test_head_matmul_topk(hip, oracle, rows, m):
    """Q6_K output head + top-40 per column, candidates only (config 4 at reduced rows)."""
    print(f"head rows={rows} m={m}", flush=True)
    k_in = 2560
    seed = S.derive(S.config_seed(4), "head", rows, m)
    w = S.q6_k_blocks(seed, rows, k_in)
    x = S.activations(seed, m, k_in)
    h = hip.createHipQuantizedWeightHandle("Q6_K", w, k_in, rows)
    try:
        got = hip.matMulQuantizedHipResidentTopK(h, x, k_in, m, 40)
    finally:
        hip.releaseHipQuantizedWeightHandle(h)
    logits = oracle.matmul(3, w, x, rows, threads=8)
    _check_rows(got, logits, 40, oracle)


def test_geglu_bit_exact(hip, oracle):
    n = 1 << 20
    seed = S.derive(S.BASE_SEED, "geglu")
    gate = (S.activations(seed, 1, n)[0] * 3.0).astype(np.float32)
    up = S.activations(S.derive(seed, 1), 1, n)[0]
    special = np.array([0.0, -0.0, 1.0, -1.0, 10.0, -10.0, 9.999999, -9.999999, 10.000001, -10.000001,
                        5.960464477539063e-08, -5.960464477539063e-08, 2.9802322387695312e-08, 1e-30, -1e-40,
                        3.0, -3.0, 0.5, 7.25, 65504.0, -65504.0, 1e6], dtype=np.float32)
    gate[: special.size] = special
    up[: special.size] = np.linspace(-2, 2, special.size).astype(np.float32)
    got = hip.gegluHip(gate, up)
    ref = oracle.geglu(gate, up)
    diff = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert diff.size == 0, (diff[:5], gate[diff[:5]], got[diff[:5]], ref[diff[:5]])


def test_geglu_every_f16_input(hip, oracle):
    """The GeGLU launches read gelu from a table of its value at each f16
    pattern (gelu rounds its input to f16 first).  Every one of the 65536
    patterns as gate, each beside up = 1 (the table entry itself), a NaN
    payload and neighbours just inside and outside +-10 (the range checks
    run on the unrounded input), against the oracle bit for bit."""
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nudge = np.array([np.nextafter(np.float32(10.0), np.float32(0.0)), np.nextafter(np.float32(-10.0), np.float32(0.0)),
                      np.float32(9.9951171875), np.float32(-9.9951171875), np.float32(9.998), np.float32(-9.998)],
                     dtype=np.float32)
    nan = np.array([0x7FC00001, 0xFFC12345], dtype=np.uint32).view(np.float32)
    gate = np.concatenate([pats, pats, nudge, nan]).astype(np.float32)
    up = np.concatenate([np.ones(65536, np.float32), np.full(65536, -1.75, np.float32),
                         np.full(nudge.size + nan.size, 0.625, np.float32)])
    got = hip.gegluHip(gate, up)
    ref = oracle.geglu(gate, up)
    diff = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert diff.size == 0, (diff[:5], gate[diff[:5]], got[diff[:5]], ref[diff[:5]])


@pytest.mark.parametrize("kernel", [0, 1, 2, 3, 6], ids=["auto", "valu-fused", "mfma", "half", "wide"])
@pytest.mark.parametrize("rows,k,m", [(600, 2560, 1), (610, 2560, 3), (60, 10240, 1), (10240, 2560, 1),
                                      (777, 2560, 4), (1, 2560, 2)])
def test_matmul_geglu_bit_exact(hip, oracle, kernel, rows, k, m):
    """gate/up + GeGLU (layers.ts:432-456) through hp_hip_matmul_geglu: the
    fused single launch (vector ALU, up to four columns) and the
    two-launch path of the other kernels against the oracle."""
    print(f"matmul_geglu kernel={kernel} rows={rows} k={k} m={m}", flush=True)
    seed = S.derive(S.BASE_SEED, "ffn-geglu", rows, k, m)
    wg = S.q4_k_blocks(S.derive(seed, "g"), rows, k)
    wu = S.q4_k_blocks(S.derive(seed, "u"), rows, k)
    x = S.activations(seed, m, k)
    hg = hip.createHipQuantizedWeightHandle("Q4_K", wg, k, rows)
    hu = hip.createHipQuantizedWeightHandle("Q4_K", wu, k, rows)
    hip.setMatvecKernel(kernel)
    try:
        got = hip.matMulGegluHipResident(hg, hu, x, k, m).reshape(m, rows)
    finally:
        hip.setMatvecKernel(0)
        hip.releaseHipQuantizedWeightHandle(hg)
        hip.releaseHipQuantizedWeightHandle(hu)
    g = oracle.matmul(1, wg, x, rows)
    u = oracle.matmul(1, wu, x, rows)
    ref = oracle.geglu(g.reshape(-1), u.reshape(-1)).reshape(m, rows)
    bad = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, (bad[:5], got.reshape(-1)[bad[:5]], ref.reshape(-1)[bad[:5]])
