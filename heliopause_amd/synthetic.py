"""Deterministic synthetic GGUF super-blocks and activations.

Every workload in the tests and the benchmark is generated here from one
64-bit seed, so the HIP path and the CPU checker always see identical bytes.

Generator: SplitMix64 (counter form: draw ``i`` of stream ``s`` is
``mix(s + (i + 1) * 0x9E3779B97F4A7C15)``), N(0,1) by Box-Muller in f64.
Each tensor field draws from its own stream ``derive(seed, label)``.

Block distributions (the benchmark's workload definitions):

* Q4_K (144 B, ggml layout ``packages/engine/wasm-kernels/src/lib.rs:1630-1664``):
  quants uniform 0..15 (uniform random bytes), 6-bit scales and mins uniform
  0..63 packed as the inverse of ``get_scale_min_k4`` (lib.rs:2249-2259),
  ``d`` and ``dmin`` = f16(|N(0,1)| * 0.01).
* Q6_K (210 B, lib.rs:1709-1744): 6-bit quants uniform 0..63 (uniform random
  ql/qh bytes), int8 scales uniform -32..31, ``d`` = f16(|N(0,1)| * 0.005).
* activations: f32 N(0,1).
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
MASK64 = (1 << 64) - 1

Q4_K_BYTES = 144
Q6_K_BYTES = 210
BASE_SEED = 0x48454C494F50  # "HELIOP"


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _mix_int(z: int) -> int:
    z &= MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def derive(seed: int, *labels) -> int:
    """Sub-stream seed for ``labels`` (ints or strings) under ``seed``."""
    s = seed & MASK64
    for lab in labels:
        if isinstance(lab, str):
            v = 0
            for ch in lab.encode():
                v = (v * 131 + ch) & MASK64
        else:
            v = int(lab) & MASK64
        s = _mix_int(s ^ _mix_int(v + 0x9E3779B97F4A7C15))
    return s


_SYNTH = None


def _synth_lib():
    """The C form of the stream (libhp_synth.so, built beside this file), or
    None; both give the same words."""
    global _SYNTH
    if _SYNTH is None:
        import ctypes
        from pathlib import Path

        path = Path(__file__).resolve().parent / "libhp_synth.so"
        _SYNTH = False
        if path.exists():
            try:
                L = ctypes.CDLL(str(path))
                L.hp_synth_splitmix64.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                                  ctypes.c_void_p, ctypes.c_int]
                L.hp_synth_splitmix64.restype = ctypes.c_int
                _SYNTH = L
            except OSError:
                _SYNTH = False
    return _SYNTH or None


def splitmix64_numpy(seed: int, n: int, start: int = 0) -> np.ndarray:
    """The stream's definition: draw i (counted from ``start``) is
    mix(seed + ((start + i + 1) mod 2^64) * GOLDEN), all mod 2^64."""
    with np.errstate(over="ignore"):
        i = np.arange(n, dtype=np.uint64) + np.uint64((start + 1) & MASK64)
        z = np.uint64(seed & MASK64) + i * GOLDEN
        return _mix(z)


def splitmix64(seed: int, n: int, start: int = 0, threads: int | None = None) -> np.ndarray:
    """Draws ``start .. start+n-1`` of the SplitMix64 stream ``seed`` (the C
    form for large draws when libhp_synth.so is built; the numpy form when
    it is not, or when the C call reports an error)."""
    L = _synth_lib() if n >= 4096 else None
    if L is not None:
        import os

        out = np.empty(n, dtype=np.uint64)
        t = threads if threads is not None else min(16, os.cpu_count() or 1)
        if L.hp_synth_splitmix64(seed & MASK64, start & MASK64, n, out.ctypes.data, t) == 0:
            return out
    return splitmix64_numpy(seed, n, start)


def random_bytes(seed: int, nbytes: int) -> np.ndarray:
    words = splitmix64(seed, (nbytes + 7) // 8)
    return words.view(np.uint8)[:nbytes]


def normal(seed: int, n: int) -> np.ndarray:
    """N(0,1) by Box-Muller (f64), returned as f64."""
    pairs = (n + 1) // 2
    w = splitmix64(seed, 2 * pairs)
    u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n]


def activations(seed: int, m: int, k: int) -> np.ndarray:
    """f32 N(0,1) activations, shape [m][k]."""
    return normal(derive(seed, "x"), m * k).astype(np.float32).reshape(m, k)


def pack_scale_min_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack 6-bit (scale, min) x8 into the 12 bytes get_scale_min_k4 reads.

    For j < 4: ``q[j] = sc[j] | (sc[j+4] >> 4) << 6``,
    ``q[j+4] = mn[j] | (mn[j+4] >> 4) << 6``,
    ``q[j+8] = (sc[j+4] & 15) | (mn[j+4] & 15) << 4``.
    """
    sc = np.asarray(sc, dtype=np.uint8)
    mn = np.asarray(mn, dtype=np.uint8)
    q = np.empty(sc.shape[:-1] + (12,), dtype=np.uint8)
    lo_s, hi_s = sc[..., :4], sc[..., 4:]
    lo_m, hi_m = mn[..., :4], mn[..., 4:]
    q[..., 0:4] = lo_s | ((hi_s >> 4) << 6)
    q[..., 4:8] = lo_m | ((hi_m >> 4) << 6)
    q[..., 8:12] = (hi_s & 15) | ((hi_m & 15) << 4)
    return q


def _f16_bytes(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint8).reshape(values.shape + (2,))


def q4_k_blocks(seed: int, rows: int, k: int, d_scale: float = 0.01) -> np.ndarray:
    """Q4_K weights [rows][k/256*144] u8 with the documented distribution."""
    assert k % 256 == 0
    nb = rows * (k // 256)
    out = np.empty((nb, Q4_K_BYTES), dtype=np.uint8)
    z = normal(derive(seed, "q4k.d"), 2 * nb).reshape(nb, 2)
    out[:, 0:2] = _f16_bytes(np.abs(z[:, 0]) * d_scale)
    out[:, 2:4] = _f16_bytes(np.abs(z[:, 1]) * d_scale)
    sm = random_bytes(derive(seed, "q4k.scales"), 16 * nb).reshape(nb, 16) & 63
    out[:, 4:16] = pack_scale_min_k4(sm[:, :8], sm[:, 8:])
    out[:, 16:144] = random_bytes(derive(seed, "q4k.qs"), 128 * nb).reshape(nb, 128)
    return out.reshape(rows, -1)


def q6_k_blocks(seed: int, rows: int, k: int, d_scale: float = 0.005) -> np.ndarray:
    """Q6_K weights [rows][k/256*210] u8 with the documented distribution."""
    assert k % 256 == 0
    nb = rows * (k // 256)
    out = np.empty((nb, Q6_K_BYTES), dtype=np.uint8)
    out[:, 0:192] = random_bytes(derive(seed, "q6k.q"), 192 * nb).reshape(nb, 192)
    sc = (random_bytes(derive(seed, "q6k.scales"), 16 * nb).reshape(nb, 16) & 63).astype(np.int16) - 32
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    z = normal(derive(seed, "q6k.d"), nb)
    out[:, 208:210] = _f16_bytes(np.abs(z) * d_scale)
    return out.reshape(rows, -1)


def weight_blocks(type_name: str, seed: int, rows: int, k: int) -> np.ndarray:
    if type_name == "Q4_K":
        return q4_k_blocks(seed, rows, k)
    if type_name == "Q6_K":
        return q6_k_blocks(seed, rows, k)
    raise ValueError(f"unsupported type {type_name}")


def config_seed(config_id: int) -> int:
    return BASE_SEED + config_id
