"""GPU parity: Q4_K/Q6_K dequantisation and Q8_K matvec vs the oracle.

Bar: bit-exact (the runner replays the reference's integer sums and its f32
tail order, lib.rs:2116-2172 / 1923-1968), compared as raw f32 bit patterns.
"""
import numpy as np
import pytest

from heliopause_amd import synthetic as S

pytestmark = pytest.mark.gpu

TYPES = {"Q4_K": 1, "Q6_K": 3}


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _weights(type_name, seed, rows, k):
    return S.weight_blocks(type_name, seed, rows, k)


@pytest.fixture(params=[1, 2, 3, 4, 6, 7, 8], ids=["valu", "mfma", "half", "prefill", "wide", "wide-whole",
                                                   "wide-half"])
def kernel(request, hip):
    """Runs the test with the vector-ALU, the matrix-core, the half-split
    vector-ALU, the bit-exact prefill and the wide (one workgroup per block of
    rows) matvec, the last with whole and with half row-blocks per thread; a
    launch a forced kernel does not take (the wide kernel: more than four
    columns, mixed types; half row-blocks: more than two columns) runs the
    automatic choice."""
    hip.setMatvecKernel(request.param)
    yield request.param
    hip.setMatvecKernel(0)


@pytest.mark.parametrize("type_name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("rows,k", [(1, 256), (7, 2560), (100, 512), (13, 10240), (64, 2048)])
def test_dequantize_bit_exact(hip, oracle, type_name, rows, k):
    print(f"dequant {type_name} rows={rows} k={k}", flush=True)
    w = _weights(type_name, S.derive(S.BASE_SEED, "deq", rows, k), rows, k)
    h = hip.createHipQuantizedWeightHandle(type_name, w, k, rows)
    try:
        got = hip.dequantizeHipResident(h, 0, rows)
        ref = np.stack([oracle.dequantize(TYPES[type_name], w[r], k) for r in range(rows)])
        assert np.array_equal(_bits(got), _bits(ref))
        if rows > 3:
            part = hip.dequantizeHipResident(h, 2, rows - 3)
            assert np.array_equal(_bits(part), _bits(ref[2:rows - 1]))
    finally:
        hip.releaseHipQuantizedWeightHandle(h)


@pytest.mark.parametrize("type_name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("rows,k,m", [(1, 256, 1), (7, 2560, 1), (61, 2560, 3), (100, 512, 8), (13, 10240, 2),
                                      (64, 2048, 4), (5, 768, 11), (130, 2560, 5), (3, 4096, 1)])
def test_matmul_bit_exact(hip, oracle, kernel, type_name, rows, k, m):
    print(f"matmul kernel={kernel} {type_name} rows={rows} k={k} m={m}", flush=True)
    seed = S.derive(S.BASE_SEED, "mm", type_name, rows, k, m)
    w = _weights(type_name, seed, rows, k)
    x = S.activations(seed, m, k)
    h = hip.createHipQuantizedWeightHandle(type_name, w, k, rows)
    try:
        got = hip.matMulQuantizedHipResident(h, x, k, rows, m).reshape(m, rows)
        ref = oracle.matmul(TYPES[type_name], w, x, rows)
        assert np.array_equal(_bits(got), _bits(ref)), np.abs(got - ref).max()
    finally:
        hip.releaseHipQuantizedWeightHandle(h)


@pytest.mark.parametrize("specs", [[("Q4_K", 96), ("Q4_K", 40), ("Q6_K", 40)],
                                   [("Q6_K", 97), ("Q4_K", 41), ("Q4_K", 1), ("Q6_K", 8)],
                                   [("Q4_K", 301), ("Q4_K", 3), ("Q4_K", 77)],
                                   [("Q6_K", 5), ("Q6_K", 260), ("Q6_K", 31), ("Q6_K", 2)]],
                         ids=["qkv", "ragged4", "q4x3", "q6x4"])
def test_multi_mixed_types_bit_exact(hip, oracle, kernel, specs):
    """Q (Q4_K) + K (Q4_K) + V (Q6_K) in one launch sharing one Q8_K (lib.rs:300-426);
    ragged row counts put rows of two weights (of either type) in one
    half-split unit."""
    k = 2560
    for m in (1, 2, 4):
        print(f"multi kernel={kernel} m={m} specs={specs}", flush=True)
        seed = S.derive(S.BASE_SEED, "multi", m, len(specs))
        ws = [_weights(t, S.derive(seed, i), r, k) for i, (t, r) in enumerate(specs)]
        x = S.activations(seed, m, k)
        hs = [hip.createHipQuantizedWeightHandle(t, w, k, r) for (t, r), w in zip(specs, ws)]
        try:
            outs = hip.matMulQuantizedHipResidentMulti(hs, x, k, m)
            refs = oracle.matmul_multi([TYPES[t] for t, _ in specs], ws, x, [r for _, r in specs])
            for got, ref, (t, r) in zip(outs, refs, specs):
                assert np.array_equal(_bits(got.reshape(m, r)), _bits(ref)), t
            singles = [hip.matMulQuantizedHipResident(h, x, k, r, m) for h, (t, r) in zip(hs, specs)]
            for got, single in zip(outs, singles):
                assert np.array_equal(_bits(got), _bits(single))
        finally:
            for h in hs:
                hip.releaseHipQuantizedWeightHandle(h)


def test_special_inputs(hip, oracle, kernel):
    """All-zero columns, first-index |x| ties, a huge spike and denormal-scale inputs."""
    k, rows = 2560, 37
    for type_name in ("Q4_K", "Q6_K"):
        w = _weights(type_name, S.derive(S.BASE_SEED, "special", type_name), rows, k)
        x = np.zeros((5, k), dtype=np.float32)
        x[1, 5], x[1, 9] = 2.0, -2.0
        x[1, 300], x[1, 301] = -3.5, 3.5
        x[2] = S.activations(7, 1, k)[0]
        x[2, 1000] = 1e30
        x[3] = S.activations(8, 1, k)[0] * 1e-39
        x[4, ::7] = 2.5
        h = hip.createHipQuantizedWeightHandle(type_name, w, k, rows)
        try:
            got = hip.matMulQuantizedHipResident(h, x, k, rows, 5).reshape(5, rows)
            ref = oracle.matmul(TYPES[type_name], w, x, rows)
            assert np.array_equal(_bits(got), _bits(ref)), type_name
        finally:
            hip.releaseHipQuantizedWeightHandle(h)


@pytest.mark.parametrize("type_name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("rows,k", [(2560, 10240), (37, 10240), (700, 2560), (1, 256), (300, 4096)])
def test_wide_kernel_columns(hip, oracle, type_name, rows, k):
    """The wide kernel at one to four columns, with the special inputs of
    test_special_inputs (an all-zero column, first-index |x| ties, a huge
    spike, denormal scales): one launch per column count, every column
    compared with the oracle bit for bit."""
    seed = S.derive(S.BASE_SEED, "wide", type_name, rows, k)
    w = _weights(type_name, seed, rows, k)
    x = S.activations(seed, 4, k)
    x[1, :] = 0.0
    x[1, 5], x[1, 9], x[1, 300 % k], x[1, 301 % k] = 2.0, -2.0, -3.5, 3.5
    x[2, k // 3] = 1e30
    x[3] *= 1e-39
    h = hip.createHipQuantizedWeightHandle(type_name, w, k, rows)
    try:
        ref = oracle.matmul(TYPES[type_name], w, x, rows, threads=8)
        for sel in (6, 7, 8):  # automatic split, whole and half row-blocks per thread
            hip.setMatvecKernel(sel)
            for m in (1, 2, 3, 4):
                print(f"wide sel={sel} {type_name} rows={rows} k={k} m={m}", flush=True)
                got = hip.matMulQuantizedHipResident(h, x[:m], k, rows, m).reshape(m, rows)
                assert np.array_equal(_bits(got), _bits(ref[:m])), (sel, m)
    finally:
        hip.setMatvecKernel(0)
        hip.releaseHipQuantizedWeightHandle(h)


def _q6k_full_range_scales(seed, rows, k):
    """Q6_K blocks whose 16 int8 sub-block scales span -128..127 (as in
    quantised model files, where a block's largest sub-block takes -128),
    with +-127 and -67 planted in the first block."""
    w = S.q6_k_blocks(seed, rows, k).reshape(-1, 210).copy()
    w[:, 192:208] = S.random_bytes(S.derive(seed, "q6k.fullscales"), 16 * w.shape[0]).reshape(-1, 16)
    w[0, 192:195] = np.array([127, -127, -67], dtype=np.int8).view(np.uint8)
    return w.reshape(rows, -1)


@pytest.mark.parametrize("kernel_id", [0, 1, 2, 3, 4, 5, 6, 7, 8],
                         ids=["auto", "valu", "mfma", "half", "prefill", "fast", "wide", "wide-whole", "wide-half"])
def test_q6k_full_range_scales(hip, oracle, kernel_id):
    """Q6_K scales beyond +-66 make sc * (q - 32) inexact as an f16 matrix-core
    operand; such weights run the vector-ALU kernels under every selector, so
    the results stay bit-exact (alone and in a launch with Q4_K weights) at
    decode and prefill column counts."""
    k = 2560
    seed = S.derive(S.BASE_SEED, "q6kfull", kernel_id)
    w6 = _q6k_full_range_scales(seed, 300, k)
    w4 = _weights("Q4_K", S.derive(seed, 1), 64, k)
    h6 = hip.createHipQuantizedWeightHandle("Q6_K", w6, k, 300)
    h4 = hip.createHipQuantizedWeightHandle("Q4_K", w4, k, 64)
    hip.setMatvecKernel(kernel_id)
    try:
        for m in (1, 4, 8, 64):
            print(f"q6k full-range kernel={kernel_id} m={m}", flush=True)
            x = S.activations(S.derive(seed, m), m, k)
            ref6 = oracle.matmul(3, w6, x, 300, threads=8)
            got = hip.matMulQuantizedHipResident(h6, x, k, 300, m).reshape(m, 300)
            assert np.array_equal(_bits(got), _bits(ref6)), (m, np.abs(got - ref6).max())
            outs = hip.matMulQuantizedHipResidentMulti([h4, h6], x, k, m)
            assert np.array_equal(_bits(outs[1].reshape(m, 300)), _bits(ref6)), m
            assert np.array_equal(_bits(outs[0].reshape(m, 64)), _bits(oracle.matmul(1, w4, x, 64))), m
    finally:
        hip.setMatvecKernel(0)
        hip.releaseHipQuantizedWeightHandle(h6)
        hip.releaseHipQuantizedWeightHandle(h4)


def test_shape_errors(hip):
    k, rows = 512, 8
    w = _weights("Q4_K", 1, rows, k)
    assert hip.createHipQuantizedWeightHandle("Q5_K", w, k, rows) is None
    with pytest.raises(ValueError):
        hip.createHipQuantizedWeightHandle("Q4_K", w[:, :144], 300, rows)
    with pytest.raises(ValueError):
        hip.createHipQuantizedWeightHandle("Q4_K", w.reshape(-1)[:-1], k, rows)
    h = hip.createHipQuantizedWeightHandle("Q4_K", w, k, rows)
    try:
        with pytest.raises(ValueError):
            hip.matMulQuantizedHipResident(h, np.zeros(k + 1, np.float32), k, rows, 1)
        with pytest.raises(ValueError):
            hip.matMulQuantizedHipResident(h, np.zeros(k, np.float32), k, rows + 1, 1)
        assert hip.matMulQuantizedHipResident(h, np.zeros(0, np.float32), k, rows, 0).size == 0
        assert hip.matMulQuantizedHipResidentMulti([h], np.zeros(k, np.float32), k, 1) is None
    finally:
        hip.releaseHipQuantizedWeightHandle(h)
    code = hip.lib().hp_hip_weight_release(h.handle)
    assert code == hip.HP_ERR_HANDLE


@pytest.mark.parametrize("m,k", [(1, 256), (3, 2560), (2, 10240)])
def test_q8k_bit_exact(hip, oracle, m, k):
    """The in-kernel Q8_K quantisation (lib.rs:1774-1811) vs the oracle, all outputs."""
    print(f"q8k m={m} k={k}", flush=True)
    x = S.activations(S.derive(S.BASE_SEED, "q8k", m, k), m, k)
    base = 0
    if k >= 512:
        x[0, :256] = 0.0                  # all-zero block
        base = 256
    x[0, base + 3], x[0, base + 7] = 9.0, -9.0  # |x| tie -> first index wins
    x[-1, -1] = np.nan                    # NaN never selected as max; quantises to 127
    x[-1, 5] = 2.5 * 127 / 127            # exercise ties away from zero at is*x = .5
    qs, d, bs = hip.quantizeQ8KHip(x, k, m)
    rq, rd, rb = oracle.quantize_q8_k(x)
    assert np.array_equal(qs, rq)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(bs, rb)
