"""Pins the oracle's Q8_K quantisation and Q4_K/Q6_K vec-dots (CPU only).

Q8_K (lib.rs:1774-1811) is checked on hand-built special cases and against
an independent vectorised statement written here (first index of max |x|,
f32 divide, round half away from zero computed exactly in f64).  The vec-dot
integers are checked per accumulator lane against a brute-force decode of
the logical block elements, and the f32 results against an f64 dot of
dequantised weights with the dequantised Q8_K input.  Matmul API behaviour
follows lib.rs:224-426 (status codes, multi == separate calls) and the
thread pool's sharding (thread-pool.ts:410-443: sharded == unsharded).
"""
import numpy as np
import pytest

from heliopause_amd import synthetic as S

Q4K, Q6K = 1, 3


def q8k_reference(x):
    """Independent vectorised Q8_K of rows of x (f32)."""
    x = np.asarray(x, np.float32).reshape(x.shape[0], -1, 256)
    a = np.abs(x)
    first = np.argmax(a, axis=2)  # first occurrence of the maximum
    mx = np.take_along_axis(x, first[..., None], axis=2)[..., 0]
    amax = a.max(axis=2)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        inv = (np.float32(-127.0) / mx).astype(np.float32)
        p = (inv[..., None] * x).astype(np.float32).astype(np.float64)
        r = np.sign(p) * np.floor(np.abs(p) + 0.5)  # exact: ties away from zero
        r = np.where(np.isnan(r), 127.0, np.minimum(r, 127.0))
        q = np.clip(r, -128, 127).astype(np.int8)
        d = (np.float32(1.0) / inv).astype(np.float32)
    q[amax == 0] = 0
    d = np.where(amax == 0, np.float32(0), d).astype(np.float32)
    bs = q.reshape(x.shape[0], -1, 8, 32).astype(np.int32).sum(axis=3).astype(np.int16)
    return q.reshape(x.shape[0], -1), d, bs.reshape(x.shape[0], -1)


def test_q8k_special_cases(oracle):
    x = np.zeros((1, 512), np.float32)
    x[0, 256 + 5], x[0, 256 + 9] = 2.0, -2.0
    qs, d, bs = oracle.quantize_q8_k(x)
    assert not qs[0, :256].any() and d[0, 0] == 0.0 and not bs[0, :8].any()  # amax == 0
    # first maximum is +2: is = -63.5, d < 0
    assert qs[0, 256 + 5] == -127 and qs[0, 256 + 9] == 127 and d[0, 1] < 0
    x[0, 256 + 5], x[0, 256 + 9] = -2.0, 2.0
    qs, d, _ = oracle.quantize_q8_k(x)
    assert qs[0, 256 + 5] == -127 and qs[0, 256 + 9] == 127 and d[0, 1] > 0
    # ties away from zero: max = -127 gives is = 1
    y = np.zeros((1, 256), np.float32)
    y[0, :6] = [-127.0, 2.5, -2.5, 0.5, -0.5, 1.5]
    qs, d, _ = oracle.quantize_q8_k(y)
    assert list(qs[0, :6]) == [-127, 3, -3, 1, -1, 2] and d[0, 0] == 1.0
    # NaN is never the max and quantises to min(NaN, 127) = 127
    z = np.ones((1, 256), np.float32)
    z[0, 3] = np.nan
    qs, _, _ = oracle.quantize_q8_k(z)
    assert qs[0, 3] == 127 and qs[0, 0] == -127


def test_q8k_matches_independent_statement(oracle):
    x = S.activations(11, 3, 2560)
    x[1, 100:356] = 0.0
    x[2, 7] = -1e20
    qs, d, bs = oracle.quantize_q8_k(x)
    rq, rd, rb = q8k_reference(x)
    assert np.array_equal(qs, rq) and np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(bs, rb)
    # reconstruction bound and the max element at -127
    recon = (qs.astype(np.float64).reshape(3, -1, 256) * d[..., None]).reshape(3, -1)
    nz = np.repeat(d != 0, 256, axis=1)
    err = np.abs(recon - x)
    assert (err[nz] <= np.repeat(np.abs(d), 256, axis=1)[nz] * 0.5000001 + 1e-30).all()


def decode_q4k(blk):
    """(sc[j], mn[j], q[e]) of a Q4_K block by the format description."""
    sc, mn = [], []
    s = blk[4:16]
    for j in range(8):
        if j < 4:
            sc.append(s[j] & 63)
            mn.append(s[j + 4] & 63)
        else:
            sc.append((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4))
            mn.append((s[j + 4] >> 4) | ((s[j] >> 6) << 4))
    e = np.arange(256)
    j = e // 32
    q = (blk[16 + 32 * (j // 2) + e % 32] >> (4 * (j % 2))) & 15
    return np.array(sc, np.int64), np.array(mn, np.int64), q.astype(np.int64)


def decode_q6k(blk):
    e = np.arange(256)
    h, t, l = e // 128, (e % 128) // 32, e % 32
    lo = (blk[64 * h + l + 32 * (t & 1)] >> (4 * (t >> 1))) & 15
    hi = (blk[128 + 32 * h + l] >> (2 * t)) & 3
    q = (lo | (hi << 4)).astype(np.int64) - 32
    sc = blk[192:208].view(np.int8).astype(np.int64)
    return sc, q


@pytest.mark.parametrize("type_id", [Q4K, Q6K])
def test_block_integers_per_lane(oracle, type_id):
    rng = np.random.default_rng(12)
    for trial in range(40):
        w = (S.q4_k_blocks if type_id == Q4K else S.q6_k_blocks)(trial, 1, 256)[0]
        x = S.activations(trial + 100, 1, 256)
        qs, d, bs = oracle.quantize_q8_k(x)
        q8 = qs[0].astype(np.int64)
        aux, sumi = oracle.block_ints(type_id, w, qs[0], bs[0])
        e = np.arange(256)
        if type_id == Q4K:
            sc, mn, q = decode_q4k(w)
            want = [int((sc[e // 32] * q * q8)[e % 8 == l].sum()) for l in range(8)]
            assert sumi == int((bs[0].astype(np.int64) * mn).sum())
        else:
            sc, q = decode_q6k(w)
            want = [int((sc[e // 16] * q * q8)[e % 8 == l].sum()) for l in range(8)]
        assert list(aux) == want


@pytest.mark.parametrize("type_id,k", [(Q4K, 2560), (Q6K, 2560), (Q4K, 10240), (Q6K, 10240)])
def test_vec_dot_against_f64(oracle, type_id, k):
    rows, m = 24, 3
    w = (S.q4_k_blocks if type_id == Q4K else S.q6_k_blocks)(k + type_id, rows, k)
    x = S.activations(k + 7, m, k)
    out = oracle.matmul(type_id, w, x, rows)
    qs, d, _ = oracle.quantize_q8_k(x)
    xd = (qs.astype(np.float64).reshape(m, -1, 256) * d[..., None]).reshape(m, k)
    W = np.stack([oracle.dequantize(type_id, w[r], k) for r in range(rows)]).astype(np.float64)
    exact = xd @ W.T
    scale = np.abs(xd) @ np.abs(W).T
    assert (np.abs(out - exact) <= 2e-6 * scale + 1e-30).all()


def test_multi_threaded_and_status(oracle):
    k = 2560
    specs = [(Q4K, 40), (Q4K, 13), (Q6K, 29)]
    ws = [(S.q4_k_blocks if t == Q4K else S.q6_k_blocks)(i, r, k) for i, (t, r) in enumerate(specs)]
    x = S.activations(99, 4, k)
    singles = [oracle.matmul(t, w, x, r) for (t, r), w in zip(specs, ws)]
    multi = oracle.matmul_multi([t for t, _ in specs], ws, x, [r for _, r in specs])
    for a, b in zip(singles, multi):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for threads in (2, 3, 8):
        sh = oracle.matmul_multi([t for t, _ in specs], ws, x, [r for _, r in specs], threads=threads)
        for a, b in zip(singles, sh):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    w = ws[0]
    # lib.rs:240-247: input/output lengths are checked before the type
    assert oracle.matmul_status(2, w, x[:1], k, 40, 1)[0] == oracle.ERR_TYPE
    assert oracle.matmul_status(2, w, x[:1, :-1], k, 40, 1)[0] == oracle.ERR_SHAPE
    assert oracle.matmul_status(Q4K, w, x[:1], k, 40, 1, output_len=39)[0] == oracle.ERR_SHAPE
    assert oracle.matmul_status(Q4K, w[:, :-1], x[:1], k, 40, 1)[0] == oracle.ERR_SHAPE
    assert oracle.matmul_status(Q4K, w, x[:1], 2500, 40, 1, output_len=40)[0] == oracle.ERR_SHAPE
    st, out = oracle.matmul_status(Q4K, w, np.zeros(0, np.float32), k, 40, 0)
    assert st == oracle.OK and out.size == 0
