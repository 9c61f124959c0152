"""Pins the oracle's scalar conversions and GGUF block formats (CPU only).

Checks: the reference's own known-answer tests (quant.test.ts:12-22, 58-66),
exhaustive comparison of f16 decoding with IEEE half (numpy), the TS f32->f16
rounding against IEEE round-to-nearest-even outside its documented flush and
saturation ranges, the 6-bit scale packing as a bijection, and dequantisation
of blocks assembled from logical fields by a packer written here from the
format description, with the closed-form f32 result.
"""
import math

import numpy as np
import pytest

from heliopause_amd import synthetic as S

Q4K, Q6K = 1, 3


def test_f16_known_answers(oracle):
    # quant.test.ts:12-17
    assert oracle.f16_to_f32(0x0000) == 0.0
    assert oracle.f16_to_f32(0x3C00) == 1.0
    assert oracle.f16_to_f32(0xC000) == -2.0
    assert oracle.f16_to_f32(0x7C00) == np.inf
    assert oracle.f16_to_f64_ts(0x3C00) == 1.0
    assert oracle.f16_to_f64_ts(0xC000) == -2.0
    assert oracle.f16_to_f64_ts(0x7C00) == np.inf


def test_f16_decode_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ieee = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32_bits(int(b)) for b in bits], dtype=np.uint32)
    nan = np.isnan(ieee)
    assert np.array_equal(got[~nan], ieee[~nan].view(np.uint32))
    # NaN payload kept (lib.rs:2525-2527): sign | 0x7f800000 | frac << 13
    b = bits[nan].astype(np.uint32)
    assert np.array_equal(got[nan], ((b & 0x8000) << 16) | 0x7F800000 | ((b & 0x3FF) << 13))
    ts = np.array([oracle.f16_to_f64_ts(int(x)) for x in bits[~nan]])
    assert np.array_equal(ts, bits[~nan].view(np.float16).astype(np.float64))


def test_f32_to_f16_ts(oracle):
    # quant.test.ts:19-22 (ties to even)
    assert oracle.f64_to_f16_ts(1 + 0.5 / 1024) == 0x3C00
    assert oracle.f64_to_f16_ts(1 + 1.5 / 1024) == 0x3C02
    rng = np.random.default_rng(1)
    e = rng.integers(-24, 16, 200000)
    v = (rng.random(200000) + 1.0) * np.exp2(e.astype(np.float64))
    v = np.where(rng.random(200000) < 0.5, -v, v).astype(np.float32)
    # add exact ties on the f16 grid
    v[:1000] = (np.arange(1000, dtype=np.float32) + 0.5) / 1024 + 1.0
    for x in v[:60000]:
        a = abs(float(x))
        got = oracle.f64_to_f16_ts(float(x))
        if a < 2.0 ** -24:
            assert got & 0x7FFF == 0
        elif a >= 65504:
            assert got & 0x7FFF == 0x7BFF
        else:
            assert got == int(np.float32(x).astype(np.float16).view(np.uint16)), x
    assert oracle.f64_to_f16_ts(float("nan")) == 0x7E00
    assert oracle.f64_to_f16_ts(float("inf")) == 0x7C00
    assert oracle.f64_to_f16_ts(-float("inf")) == 0xFC00
    assert oracle.f64_to_f16_ts(-0.0) == 0x8000
    assert oracle.f64_to_f16_ts(70000.0) == 0x7BFF


def _f16_half_away(x: float) -> int:
    """f16 bits of x rounded to nearest, ties away from zero, saturating at
    65504, flushing below 2^-25 to zero: computed exactly in f64."""
    if math.isnan(x):
        return 0x7E00
    sign = 0x8000 if math.copysign(1.0, x) < 0 else 0
    a = abs(x)
    if math.isinf(a):
        return sign | 0x7C00
    if a < 2.0 ** -25:
        return sign
    if a < 2.0 ** -14:
        return sign | int(math.floor(a / 2.0 ** -24 + 0.5))
    mant, e = math.frexp(a)  # a = mant * 2^e, mant in [0.5, 1)
    e -= 1
    m = int(math.floor(a / 2.0 ** (e - 10) + 0.5))
    if m == 2048:
        e, m = e + 1, 1024
    if e > 15:
        return sign | 0x7BFF
    return sign | ((e + 15) << 10) | (m - 1024)


def test_f32_to_f16_rust_rounds_half_up(oracle):
    # lib.rs:2534-2569 adds half an ulp before truncating (ties away)
    assert oracle.f32_to_f16_rust(1 + 0.5 / 1024) == 0x3C01
    assert oracle.f32_to_f16_rust(1.0) == 0x3C00
    assert oracle.f32_to_f16_rust(65520.0) == 0x7BFF
    rng = np.random.default_rng(3)
    e = rng.integers(-27, 17, 40000).astype(np.float64)
    v = ((rng.random(40000) + 1.0) * np.exp2(e)).astype(np.float32)
    v = np.where(rng.random(40000) < 0.5, -v, v)
    # exact ties and their neighbours, normal and subnormal
    ties = np.concatenate([(np.arange(1, 2000) + 0.5) * 2.0 ** -10, (np.arange(0, 1024) + 0.5) * 2.0 ** -24])
    ties = ties.astype(np.float32)
    extra = np.concatenate([ties, np.nextafter(ties, np.float32(0)), np.nextafter(ties, np.float32(np.inf)),
                            np.float32([65504, 65519.99, 65520, 65536, 1e9, 2.0 ** -25, 2.0 ** -26, 0.0, -0.0,
                                        np.inf, -np.inf, np.nan])])
    for x in np.concatenate([v, extra, -extra]):
        assert oracle.f32_to_f16_rust(float(x)) == _f16_half_away(float(x)), x


def test_row_bytes(oracle):
    # quant.test.ts:58-66 / tensor-reader.ts:282-293
    assert oracle.row_bytes(Q4K, 256) == 144
    assert oracle.row_bytes(Q6K, 256) == 210
    assert oracle.row_bytes(Q4K, 2560) == 1440
    assert oracle.row_bytes(Q6K, 10240) == 8400
    assert oracle.row_bytes(Q4K, 300) == 0


def test_scale_min_pack_roundtrip(oracle):
    rng = np.random.default_rng(2)
    for _ in range(200):
        sc = rng.integers(0, 64, 8).astype(np.uint8)
        mn = rng.integers(0, 64, 8).astype(np.uint8)
        q = S.pack_scale_min_k4(sc, mn).tobytes()
        for j in range(8):
            assert oracle.get_scale_min_k4(j, q) == (sc[j], mn[j])
    # unpack is a bijection on 12-byte strings: repacking restores them
    for _ in range(200):
        q = rng.integers(0, 256, 12).astype(np.uint8).tobytes()
        pairs = [oracle.get_scale_min_k4(j, q) for j in range(8)]
        sc = np.array([p[0] for p in pairs], np.uint8)
        mn = np.array([p[1] for p in pairs], np.uint8)
        assert S.pack_scale_min_k4(sc, mn).tobytes() == q


def pack_q4k(d, dmin, sc, mn, q):
    """Q4_K block from logical fields: element e in sub-block j = e // 32 sits
    in byte 16 + 32 * (j // 2) + e % 32, low nibble for even j, high for odd."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    blk[4:16] = S.pack_scale_min_k4(sc, mn)
    for e in range(256):
        j = e // 32
        blk[16 + 32 * (j // 2) + e % 32] |= np.uint8(q[e] << (4 * (j % 2)))
    return blk


def pack_q6k(d, sc, q):
    """Q6_K block from logical fields: element e = 128h + 32t + l has its low
    nibble in ql[64h + l + 32(t & 1)] (high half if t >= 2) and its top two
    bits in qh[32h + l] at bit 2t; scale sc[e // 16]."""
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        h, t, l = e // 128, (e % 128) // 32, e % 32
        blk[64 * h + l + 32 * (t & 1)] |= np.uint8((q[e] & 15) << (4 * (t >> 1)))
        blk[128 + 32 * h + l] |= np.uint8((q[e] >> 4) << (2 * t))
    blk[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


def test_q4k_dequant_closed_form(oracle):
    rng = np.random.default_rng(3)
    for _ in range(50):
        d, dmin = np.float16(abs(rng.standard_normal()) * 0.01), np.float16(abs(rng.standard_normal()) * 0.01)
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        got = oracle.dequantize(Q4K, pack_q4k(d, dmin, sc, mn, q), 256)
        j = np.arange(256) // 32
        exact = float(d) * sc[j] * q - float(dmin) * mn[j]  # f64: both products are exact
        assert np.array_equal(got, exact.astype(np.float32))  # one rounding (lib.rs:1648-1654)


def test_q6k_dequant_closed_form(oracle):
    rng = np.random.default_rng(4)
    for _ in range(50):
        d = np.float16(abs(rng.standard_normal()) * 0.005)
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(0, 64, 256)
        got = oracle.dequantize(Q6K, pack_q6k(d, sc, q), 256)
        exact = float(d) * sc[np.arange(256) // 16] * (q - 32)  # exact in f32
        assert np.array_equal(got.astype(np.float64), exact)


def test_synthetic_blocks_follow_the_distribution():
    w4 = S.q4_k_blocks(7, 64, 512).reshape(-1, 144)
    d = w4[:, 0:2].copy().view(np.float16).astype(np.float64)
    assert (d >= 0).all() and 0.003 < d.mean() < 0.012
    w6 = S.q6_k_blocks(7, 64, 512).reshape(-1, 210)
    sc = w6[:, 192:208].view(np.int8)
    assert sc.min() >= -32 and sc.max() <= 31
    x = S.activations(7, 4, 4096)
    assert abs(float(x.mean())) < 0.05 and 0.95 < float(x.std()) < 1.05
