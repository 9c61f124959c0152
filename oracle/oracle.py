"""ctypes binding to the oracle library (oracle/libhp_oracle.so).

TEST INFRASTRUCTURE ONLY: this module is the checker.  Only tests/,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it; the HIP product path never does.

Each wrapper calls one restated reference function (see hp_oracle.c for the
file:line each follows).  Arrays use the reference's layouts: activations
``[M][K]`` f32, outputs ``[M][N]`` f32, weights ``[N][row_bytes]`` u8.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libhp_oracle.so"

OK, ERR_SHAPE, ERR_HEADS, ERR_TYPE = 0, 1, 2, 3
Q4_K, Q5_K, Q6_K, IQ4_XS, Q8_0, Q4_0 = 1, 2, 3, 4, 5, 6
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}

_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i16p = ctypes.POINTER(ctypes.c_int16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


def build() -> Path:
    """Compile the oracle with its Makefile (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    _lib = _declare(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def native_lib(build_dir) -> ctypes.CDLL:
    """The oracle compiled for the running host's own ISA (-march=native, with
    the same -ffp-contract=off / -fno-fast-math numerics) into build_dir: the
    CPU baseline's native leg.  Built where it runs, since its code is only
    valid on this host's CPU."""
    out = Path(build_dir) / "libhp_oracle_native.so"
    subprocess.run([os.environ.get("CC", "gcc"), "-std=gnu11", "-O3", "-march=native", "-ffp-contract=off",
                    "-fno-fast-math", "-fPIC", "-pthread", "-shared", "-o", str(out), str(HERE / "hp_oracle.c"),
                    "-lm"], check=True, capture_output=True)
    return _declare(ctypes.CDLL(str(out)))


def _declare(L: ctypes.CDLL) -> ctypes.CDLL:
    L.hpo_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.hpo_f16_to_f32.restype = ctypes.c_float
    L.hpo_f16_to_f32_bits.argtypes = [ctypes.c_uint16]
    L.hpo_f16_to_f32_bits.restype = ctypes.c_uint32
    L.hpo_f32_to_f16_rust.argtypes = [ctypes.c_float]
    L.hpo_f32_to_f16_rust.restype = ctypes.c_uint16
    L.hpo_f16_to_f64_ts.argtypes = [ctypes.c_uint16]
    L.hpo_f16_to_f64_ts.restype = ctypes.c_double
    L.hpo_f64_to_f16_ts.argtypes = [ctypes.c_double]
    L.hpo_f64_to_f16_ts.restype = ctypes.c_uint16
    L.hpo_row_bytes.argtypes = [ctypes.c_int32, _sz]
    L.hpo_row_bytes.restype = _sz
    L.hpo_get_scale_min_k4.argtypes = [ctypes.c_int, _u8p, _u8p, _u8p]
    L.hpo_dequantize_q4_k.argtypes = [_u8p, _sz, _f32p]
    L.hpo_dequantize_q6_k.argtypes = [_u8p, _sz, _f32p]
    L.hpo_quantize_q8_k.argtypes = [_f32p, _sz, _i8p, _f32p, _i16p]
    L.hpo_vec_dot_q4_k_q8_k.argtypes = [_u8p, _sz, _i8p, _f32p, _i16p]
    L.hpo_vec_dot_q4_k_q8_k.restype = ctypes.c_float
    L.hpo_vec_dot_q6_k_q8_k.argtypes = [_u8p, _sz, _i8p, _f32p]
    L.hpo_vec_dot_q6_k_q8_k.restype = ctypes.c_float
    L.hpo_block_ints_q4_k.argtypes = [_u8p, _i8p, _i16p, _i32p, _i32p]
    L.hpo_block_ints_q6_k.argtypes = [_u8p, _i8p, _i32p]
    L.hpo_matmul_quantized.argtypes = [ctypes.c_int32, _u8p, _sz, _f32p, _sz, _sz, _sz, _sz, _f32p, _sz]
    L.hpo_matmul_quantized.restype = ctypes.c_int32
    L.hpo_matmul_quantized_threaded.argtypes = [ctypes.c_int32, _u8p, _sz, _f32p, _sz, _sz, _sz, _sz,
                                                _f32p, _sz, ctypes.c_int]
    L.hpo_matmul_quantized_threaded.restype = ctypes.c_int32
    multi = [_sz, _f32p, _sz, _sz, _sz, _i32p, ctypes.POINTER(_u8p), ctypes.POINTER(_sz),
             ctypes.POINTER(_sz), ctypes.POINTER(_f32p), ctypes.POINTER(_sz)]
    L.hpo_matmul_quantized_multi.argtypes = multi
    L.hpo_matmul_quantized_multi.restype = ctypes.c_int32
    L.hpo_matmul_quantized_multi_threaded.argtypes = multi + [ctypes.c_int]
    L.hpo_matmul_quantized_multi_threaded.restype = ctypes.c_int32
    L.hpo_gelu.argtypes = [ctypes.c_float]
    L.hpo_gelu.restype = ctypes.c_float
    L.hpo_exp.argtypes = [ctypes.c_double]
    L.hpo_exp.restype = ctypes.c_double
    L.hpo_geglu.argtypes = [_f32p, _f32p, _sz, _f32p]
    L.hpo_topk.argtypes = [_f32p, _sz, _sz, _u32p, _f32p]
    L.hpo_topk.restype = _sz
    L.hpo_softcap.argtypes = [ctypes.c_float, ctypes.c_double]
    L.hpo_softcap.restype = ctypes.c_float
    return L


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar conversions ----------------------------------------------------
def f16_to_f32(h: int) -> float:
    return lib().hpo_f16_to_f32(h)


def f16_bits_to_f32_bits(h: int) -> int:
    return int(lib().hpo_f16_to_f32_bits(h))


def f32_to_f16_rust(v: float) -> int:
    return lib().hpo_f32_to_f16_rust(v)


def f16_to_f64_ts(h: int) -> float:
    return lib().hpo_f16_to_f64_ts(h)


def f64_to_f16_ts(v: float) -> int:
    return lib().hpo_f64_to_f16_ts(v)


def row_bytes(type_id: int, elements: int) -> int:
    return lib().hpo_row_bytes(type_id, elements)


def get_scale_min_k4(j: int, q12: bytes) -> tuple[int, int]:
    q = _c(np.frombuffer(bytes(q12), dtype=np.uint8), np.uint8)
    sc = ctypes.c_uint8()
    mn = ctypes.c_uint8()
    lib().hpo_get_scale_min_k4(j, _p(q, _u8p), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


# ---- formats ------------------------------------------------------------------
def dequantize(type_id: int, data: np.ndarray, elements: int) -> np.ndarray:
    data = _c(data, np.uint8).reshape(-1)
    out = np.empty(elements, dtype=np.float32)
    fn = lib().hpo_dequantize_q4_k if type_id == Q4_K else lib().hpo_dequantize_q6_k
    fn(_p(data, _u8p), elements, _p(out, _f32p))
    return out


def quantize_q8_k(x: np.ndarray):
    """Q8_K of each row of ``x`` [M][K] -> (qs [M][K] i8, d [M][K/256] f32, bsums32 [M][K/32] i16)."""
    x = _c(np.atleast_2d(x), np.float32)
    m, k = x.shape
    qs = np.empty((m, k), dtype=np.int8)
    d = np.empty((m, k // 256), dtype=np.float32)
    bs = np.empty((m, k // 32), dtype=np.int16)
    for i in range(m):
        lib().hpo_quantize_q8_k(_p(x[i], _f32p), k, _p(qs[i], _i8p), _p(d[i], _f32p), _p(bs[i], _i16p))
    return qs, d, bs


def block_ints(type_id: int, blk: np.ndarray, qs: np.ndarray, bsums32: np.ndarray | None = None):
    blk = _c(blk, np.uint8)
    qs = _c(qs, np.int8)
    aux = np.zeros(8, dtype=np.int32)
    if type_id == Q4_K:
        bs = _c(bsums32, np.int16)
        sumi = ctypes.c_int32()
        lib().hpo_block_ints_q4_k(_p(blk, _u8p), _p(qs, _i8p), _p(bs, _i16p), _p(aux, _i32p), ctypes.byref(sumi))
        return aux, sumi.value
    lib().hpo_block_ints_q6_k(_p(blk, _u8p), _p(qs, _i8p), _p(aux, _i32p))
    return aux, 0


def vec_dot(type_id: int, row: np.ndarray, qs: np.ndarray, d: np.ndarray, bsums32: np.ndarray) -> float:
    row = _c(row, np.uint8)
    qs = _c(qs, np.int8)
    d = _c(d, np.float32)
    nb = qs.size // 256
    if type_id == Q4_K:
        bs = _c(bsums32, np.int16)
        return lib().hpo_vec_dot_q4_k_q8_k(_p(row, _u8p), nb, _p(qs, _i8p), _p(d, _f32p), _p(bs, _i16p))
    return lib().hpo_vec_dot_q6_k_q8_k(_p(row, _u8p), nb, _p(qs, _i8p), _p(d, _f32p))


# ---- matmuls ----------------------------------------------------------------
def matmul_status(type_id: int, weight: np.ndarray, x: np.ndarray, input_size: int, row_count: int,
                  column_count: int, output_len: int | None = None, threads: int = 0):
    """Raw call with the reference's shape checks; returns (status, out)."""
    weight = _c(weight, np.uint8).reshape(-1)
    x = _c(x, np.float32).reshape(-1)
    olen = row_count * column_count if output_len is None else output_len
    out = np.zeros(max(olen, 1), dtype=np.float32)
    if threads:
        st = lib().hpo_matmul_quantized_threaded(type_id, _p(weight, _u8p), weight.size, _p(x, _f32p), x.size,
                                                 input_size, row_count, column_count, _p(out, _f32p), olen,
                                                 threads)
    else:
        st = lib().hpo_matmul_quantized(type_id, _p(weight, _u8p), weight.size, _p(x, _f32p), x.size,
                                        input_size, row_count, column_count, _p(out, _f32p), olen)
    return st, out[:olen]


def matmul(type_id: int, weight: np.ndarray, x: np.ndarray, row_count: int, threads: int = 0) -> np.ndarray:
    x = _c(np.atleast_2d(x), np.float32)
    m, k = x.shape
    st, out = matmul_status(type_id, weight, x, k, row_count, m, threads=threads)
    if st != OK:
        raise RuntimeError(f"oracle matmul failed with status {st}")
    return out.reshape(m, row_count)


def matmul_multi(type_ids, weights, x: np.ndarray, row_counts, threads: int = 0,
                 library: ctypes.CDLL | None = None) -> list[np.ndarray]:
    x = _c(np.atleast_2d(x), np.float32)
    m, k = x.shape
    count = len(type_ids)
    ws = [_c(w, np.uint8).reshape(-1) for w in weights]
    outs = [np.zeros(max(r * m, 1), dtype=np.float32) for r in row_counts]
    tids = (ctypes.c_int32 * count)(*type_ids)
    wptr = (_u8p * count)(*[_p(w, _u8p) for w in ws])
    wlen = (_sz * count)(*[w.size for w in ws])
    rc = (_sz * count)(*row_counts)
    optr = (_f32p * count)(*[_p(o, _f32p) for o in outs])
    olen = (_sz * count)(*[r * m for r in row_counts])
    L = library if library is not None else lib()
    if threads:
        st = L.hpo_matmul_quantized_multi_threaded(count, _p(x, _f32p), x.size, k, m, tids, wptr, wlen, rc,
                                                   optr, olen, threads)
    else:
        st = L.hpo_matmul_quantized_multi(count, _p(x, _f32p), x.size, k, m, tids, wptr, wlen, rc, optr, olen)
    if st != OK:
        raise RuntimeError(f"oracle multi matmul failed with status {st}")
    return [o[: r * m].reshape(m, r) for o, r in zip(outs, row_counts)]


# ---- epilogues ----------------------------------------------------------------
def exp(x: float) -> float:
    """Math.exp as the JS engine computes it (fdlibm e_exp.c)."""
    return lib().hpo_exp(x)


def gelu(v: float) -> float:
    return lib().hpo_gelu(v)


def geglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = _c(gate, np.float32).reshape(-1)
    u = _c(up, np.float32).reshape(-1)
    out = np.empty_like(g)
    lib().hpo_geglu(_p(g, _f32p), _p(u, _f32p), g.size, _p(out, _f32p))
    return out.reshape(np.shape(gate))


def topk(values: np.ndarray, k: int):
    v = _c(values, np.float32).reshape(-1)
    ids = np.zeros(max(k, 1), dtype=np.uint32)
    vals = np.zeros(max(k, 1), dtype=np.float32)
    n = lib().hpo_topk(_p(v, _f32p), v.size, k, _p(ids, _u32p), _p(vals, _f32p))
    return ids[:n].copy(), vals[:n].copy()


def softcap(v: float, cap: float) -> float:
    return lib().hpo_softcap(v, cap)


def default_threads() -> int:
    """Reference default worker count, acceleration.ts:277-283."""
    return max(1, min(8, (os.cpu_count() or 4) // 2))
