"""Host mirror of heliopause's resident quantized-weight runner API, on HIP.

Mirrors ``packages/engine/src/runner/wasm/wasm-kernels.ts`` function by
function (same names with ``Wasm`` -> ``Hip``, same argument meaning, same
error behaviour), calling the C ABI in ``include/hp_hip.h`` through ctypes:

==========================================  =========================================
reference (wasm-kernels.ts)                 this module
==========================================  =========================================
``checkWasmSupport`` 1657-1675              ``checkHipSupport``
``createWasmQuantizedWeightHandle`` 520     ``createHipQuantizedWeightHandle``
``releaseWasmQuantizedWeightHandle`` 576    ``releaseHipQuantizedWeightHandle``
``wasmResidentWeightStats`` 586             ``hipResidentWeightStats``
``matMulQuantizedWasmResident`` 593         ``matMulQuantizedHipResident``
``matMulQuantizedWasmResidentMulti`` 648    ``matMulQuantizedHipResidentMulti``
``assertWasmOk`` 1882-1896                  ``assertHipOk``
``quantizedTypeId`` 1908-1923               ``quantizedTypeId``
==========================================  =========================================

Unsupported types return ``None`` (the reference's ``undefined``) so a caller
can fall back; shape errors raise.  There is no CPU fallback in this module:
if ``libhp_hip.so`` is missing or no GPU is present, calls raise.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libhp_hip.so"

HP_OK, HP_ERR_SHAPE, HP_ERR_HEADS, HP_ERR_TYPE = 0, 1, 2, 3
HP_ERR_HIP, HP_ERR_HANDLE, HP_ERR_ARG, HP_ERR_NODEV, HP_ERR_OOM = 16, 17, 18, 19, 20
HP_KERNEL_Q8K, HP_KERNEL_MATVEC, HP_KERNEL_TOPK, HP_KERNEL_GEGLU = 0, 1, 2, 3
HP_KERNEL_ATTENTION, HP_KERNEL_NORM, HP_KERNEL_SAMPLE = 4, 5, 6
KERNEL_NAMES = {HP_KERNEL_Q8K: "q8k", HP_KERNEL_MATVEC: "matvec", HP_KERNEL_TOPK: "topk", HP_KERNEL_GEGLU: "geglu",
                HP_KERNEL_ATTENTION: "attention", HP_KERNEL_NORM: "norm", HP_KERNEL_SAMPLE: "sample"}
GELU_C = float(np.sqrt(2.0 / np.pi))

TYPE_IDS = {"Q4_K": 1, "Q5_K": 2, "Q6_K": 3, "IQ4_XS": 4, "Q8_0": 5, "Q4_0": 6}
SUPPORTED = ("Q4_K", "Q6_K")
BLOCK = {"Q4_K": (256, 144), "Q6_K": (256, 210)}


class HipUnavailable(RuntimeError):
    """The HIP extension is not built or cannot be loaded."""


class HipStats(ctypes.Structure):
    _fields_ = [
        ("handle_count", ctypes.c_uint64),
        ("resident_bytes", ctypes.c_uint64),
        ("scratch_bytes", ctypes.c_uint64),
        ("matmul_calls", ctypes.c_uint64),
        ("kernel_launches", ctypes.c_uint64),
        ("device", ctypes.c_int32),
        ("compute_units", ctypes.c_int32),
    ]


_lib: Optional[ctypes.CDLL] = None
_u64 = ctypes.c_uint64
_sz = ctypes.c_size_t
_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)


def _declare(L: ctypes.CDLL) -> None:
    i32 = ctypes.c_int32
    L.hp_hip_status_string.argtypes = [i32]
    L.hp_hip_status_string.restype = ctypes.c_char_p
    L.hp_hip_last_error.argtypes = []
    L.hp_hip_last_error.restype = ctypes.c_char_p
    L.hp_hip_init.argtypes = [i32]
    L.hp_hip_shutdown.argtypes = []
    L.hp_hip_device_count.argtypes = [ctypes.POINTER(i32)]
    L.hp_hip_weight_upload.argtypes = [i32, ctypes.c_void_p, _sz, _sz, _sz, ctypes.POINTER(_u64)]
    L.hp_hip_weight_upload_device.argtypes = [i32, ctypes.c_void_p, _sz, _sz, _sz, ctypes.POINTER(_u64)]
    L.hp_hip_weight_release.argtypes = [_u64]
    L.hp_hip_weight_info.argtypes = [_u64, ctypes.POINTER(i32), ctypes.POINTER(_sz), ctypes.POINTER(_sz),
                                     ctypes.POINTER(_sz)]
    L.hp_hip_matmul.argtypes = [_u64, ctypes.c_void_p, _sz, _sz, _sz, _sz, ctypes.c_void_p, _sz]
    L.hp_hip_matmul_multi.argtypes = [_sz, ctypes.POINTER(_u64), ctypes.c_void_p, _sz, _sz, _sz,
                                      ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(_sz)]
    L.hp_hip_matmul_multi_device.argtypes = [_sz, ctypes.POINTER(_u64), ctypes.c_void_p, _sz, _sz, _sz,
                                             ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(_sz), ctypes.c_void_p]
    L.hp_hip_dequantize.argtypes = [_u64, _sz, _sz, ctypes.c_void_p, _sz]
    L.hp_hip_quantize_q8_k.argtypes = [ctypes.c_void_p, _sz, _sz, _sz, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p]
    L.hp_hip_stats.argtypes = [ctypes.POINTER(HipStats)]
    L.hp_hip_synchronize.argtypes = []
    L.hp_hip_profile.argtypes = [i32]
    L.hp_hip_profile_read.argtypes = [i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_u64)]
    for name in ("hp_hip_init", "hp_hip_shutdown", "hp_hip_device_count", "hp_hip_weight_upload",
                 "hp_hip_weight_upload_device", "hp_hip_weight_release", "hp_hip_weight_info", "hp_hip_matmul",
                 "hp_hip_matmul_multi", "hp_hip_matmul_multi_device", "hp_hip_dequantize", "hp_hip_quantize_q8_k",
                 "hp_hip_stats",
                 "hp_hip_synchronize", "hp_hip_profile", "hp_hip_profile_read"):
        getattr(L, name).restype = i32
    _declare_optional(L)


class HipSampling(ctypes.Structure):
    """hp_hip_sampling_t: resolved sampling options."""
    _fields_ = [("do_sample", ctypes.c_int32), ("top_k", ctypes.c_int32), ("temperature", ctypes.c_double),
                ("top_p", ctypes.c_double)]


class HipAttentionConfig(ctypes.Structure):
    """hp_hip_attention_config_t: attention shape, RoPE and KV ring of a layer."""
    _fields_ = [("head_count", ctypes.c_int32), ("head_count_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("rope_dims", ctypes.c_int32), ("rope_freq_base", ctypes.c_double),
                ("d_rope_freq_factors", ctypes.c_void_p), ("capacity", ctypes.c_int32),
                ("sliding_window", ctypes.c_int32), ("epsilon", ctypes.c_double)]


class HipDecodeLayer(ctypes.Structure):
    """hp_hip_decode_layer_t: one decoder layer's handles, norm weights and caches."""
    _fields_ = [("attn_q", _u64), ("attn_k", _u64), ("attn_v", _u64), ("attn_output", _u64),
                ("ffn_gate", _u64), ("ffn_up", _u64), ("ffn_down", _u64),
                ("d_attn_norm", ctypes.c_void_p), ("d_attn_q_norm", ctypes.c_void_p),
                ("d_attn_k_norm", ctypes.c_void_p), ("d_post_attention_norm", ctypes.c_void_p),
                ("d_ffn_norm", ctypes.c_void_p), ("d_post_ffw_norm", ctypes.c_void_p),
                ("layer_output_scale", ctypes.c_float), ("reserved", ctypes.c_int32),
                ("d_key_cache", ctypes.c_void_p), ("d_value_cache", ctypes.c_void_p),
                ("attention", HipAttentionConfig),
                ("inp_gate", _u64), ("proj", _u64), ("d_post_norm", ctypes.c_void_p),
                ("d_per_layer_input", ctypes.c_void_p)]


def _declare_decode(L: ctypes.CDLL) -> None:
    """Decoder-layer entry points."""
    vp, i32 = ctypes.c_void_p, ctypes.c_int32
    cfg = ctypes.POINTER(HipAttentionConfig)
    L.hp_hip_rms_norm_device.argtypes = [vp, _sz, _sz, vp, ctypes.c_double, vp, vp]
    L.hp_hip_residual_norm_device.argtypes = [vp, _sz, _sz, vp, vp, ctypes.c_float, vp, vp, vp, ctypes.c_double,
                                              vp]
    L.hp_hip_attention_prep_device.argtypes = [cfg, _sz, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    L.hp_hip_gqa_attention_device.argtypes = [cfg, _sz, vp, vp, vp, vp, vp, vp]
    L.hp_hip_decode_layers_device.argtypes = [ctypes.POINTER(HipDecodeLayer), _sz, _sz, vp, vp, vp, vp, vp]
    L.hp_hip_set_decode_fused.argtypes = [i32]
    L.hp_hip_set_fused_wait_limit.argtypes = [_u64]
    L.hp_hip_decode_fused_status.argtypes = [vp]
    L.hp_hip_set_fused_trace.argtypes = [vp, _sz]
    L.hp_hip_set_fused_trace.restype = i32
    L.hp_hip_release_stream_scratch.argtypes = [vp]
    L.hp_hip_release_stream_scratch.restype = i32
    L.hp_hip_empty_launches.argtypes = [_sz, vp]
    L.hp_hip_empty_launches.restype = i32
    for name in ("hp_hip_rms_norm_device", "hp_hip_residual_norm_device", "hp_hip_attention_prep_device",
                 "hp_hip_gqa_attention_device", "hp_hip_decode_layers_device", "hp_hip_set_decode_fused",
                 "hp_hip_set_fused_wait_limit", "hp_hip_decode_fused_status"):
        getattr(L, name).restype = i32


def _declare_optional(L: ctypes.CDLL) -> None:
    """Top-k, GeGLU, sampling and tuning entry points."""
    i32 = ctypes.c_int32
    sp = ctypes.POINTER(HipSampling)
    L.hp_hip_sample_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _sz, _sz, _sz, sp, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    L.hp_hip_sample_device.restype = i32
    L.hp_hip_matmul_topk_sample.argtypes = [_u64, ctypes.c_void_p, _sz, _sz, _sz, _sz, ctypes.c_double, sp,
                                            ctypes.POINTER(ctypes.c_uint32), ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _sz]
    L.hp_hip_matmul_topk_sample.restype = i32
    L.hp_hip_set_matvec_kernel.argtypes = [i32]
    L.hp_hip_set_matvec_kernel.restype = i32
    L.hp_hip_set_input_images.argtypes = [i32]
    L.hp_hip_set_input_images.restype = i32
    L.hp_hip_set_prefill_folds.argtypes = [i32]
    L.hp_hip_set_prefill_folds.restype = i32
    L.hp_hip_set_weight_layouts.argtypes = [i32]
    L.hp_hip_set_weight_layouts.restype = i32
    L.hp_hip_matmul_geglu.argtypes = [_u64, _u64, ctypes.c_void_p, _sz, _sz, _sz, ctypes.c_void_p, _sz]
    L.hp_hip_matmul_geglu.restype = i32
    L.hp_hip_matmul_geglu_device.argtypes = [_u64, _u64, ctypes.c_void_p, _sz, _sz, _sz, ctypes.c_void_p, _sz,
                                             ctypes.c_void_p]
    L.hp_hip_matmul_geglu_device.restype = i32
    vp = ctypes.c_void_p
    L.hp_hip_matmul_topk.argtypes = [_u64, vp, _sz, _sz, _sz, _sz, ctypes.c_double, vp, vp, _sz]
    L.hp_hip_topk.argtypes = [vp, _sz, _sz, _sz, ctypes.c_double, vp, vp, _sz]
    L.hp_hip_topk_device.argtypes = [vp, _sz, _sz, _sz, ctypes.c_double, vp, vp, vp]
    L.hp_hip_topk_device_noalloc.argtypes = [vp, _sz, _sz, _sz, ctypes.c_double, vp, vp, vp]
    L.hp_hip_geglu.argtypes = [vp, vp, _sz, vp]
    L.hp_hip_geglu_device.argtypes = [vp, vp, _sz, vp, vp]
    for name in ("hp_hip_matmul_topk", "hp_hip_topk", "hp_hip_topk_device", "hp_hip_topk_device_noalloc",
                 "hp_hip_geglu", "hp_hip_geglu_device"):
        getattr(L, name).restype = i32
    _declare_decode(L)


def lib() -> ctypes.CDLL:
    """Load libhp_hip.so (raises HipUnavailable; never falls back)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HipUnavailable(f"{LIB_PATH} is not built (run __graft_entry__.build())")
    # One HIP runtime per process.  PyTorch ships its own libamdhip64 under
    # the same soname; with torch loaded first this library binds to that
    # runtime, so torch's device pointers, streams and graphs are valid here.
    # Loaded the other way round, the process would hold two HIP runtimes
    # and torch's device initialisation fails.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    try:
        L = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the host
        raise HipUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
    _declare(L)
    _lib = L
    return L


def status_string(code: int) -> str:
    return lib().hp_hip_status_string(code).decode()


def last_error() -> str:
    return lib().hp_hip_last_error().decode()


def assertHipOk(code: int, kernel_name: str) -> None:
    """assertWasmOk (wasm-kernels.ts:1882-1896) with the HIP status codes."""
    if code == HP_OK:
        return
    if code == HP_ERR_SHAPE:
        raise ValueError(f"{kernel_name} hip shape mismatch")
    if code == HP_ERR_HEADS:
        raise ValueError(f"{kernel_name} hip head count mismatch")
    if code == HP_ERR_TYPE:
        raise TypeError(f"{kernel_name} hip unsupported type")
    detail = ""
    try:
        detail = last_error()
    except HipUnavailable:
        pass
    raise RuntimeError(f"{kernel_name} hip failed with code {code} ({detail})")


def quantizedTypeId(type_name: str) -> Optional[int]:
    """quantizedTypeId (wasm-kernels.ts:1908-1923)."""
    return TYPE_IDS.get(type_name)


def checkHipSupport() -> dict:
    """checkWasmSupport analog: {'available': bool, 'reason'?: str, 'error'?: str}."""
    try:
        L = lib()
    except HipUnavailable as exc:
        return {"available": False, "reason": "module-missing", "error": str(exc)}
    n = ctypes.c_int32(0)
    L.hp_hip_device_count(ctypes.byref(n))
    if n.value <= 0:
        return {"available": False, "reason": "device-missing"}
    return {"available": True}


@dataclass
class HipQuantizedWeightHandle:
    """WasmQuantizedWeightHandle (wasm-kernels.ts:387-397) on HBM."""

    handle: int
    type: str
    byteLength: int
    rowCount: int
    inputSize: int
    released: bool = False


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


def createHipQuantizedWeightHandle(type_name: str, weight_bytes, input_size: int,
                                   row_count: int) -> Optional[HipQuantizedWeightHandle]:
    """Upload GGUF super-blocks once into HBM (createWasmQuantizedWeightHandle, 520-574)."""
    if type_name not in TYPE_IDS or type_name not in SUPPORTED:
        return None
    if input_size <= 0 or row_count <= 0:
        raise ValueError(f"Resident quantized weight shape mismatch: inputSize={input_size} rowCount={row_count}")
    if input_size % 256 != 0:  # quantizedScaleValueCount, wasm-kernels.ts:1925-1941
        raise ValueError(f"{type_name} scale shape mismatch: {input_size}")
    if isinstance(weight_bytes, np.ndarray):
        data = np.ascontiguousarray(weight_bytes, dtype=np.uint8).reshape(-1)
    else:
        data = np.frombuffer(bytes(weight_bytes), dtype=np.uint8)
    out = _u64(0)
    code = lib().hp_hip_weight_upload(TYPE_IDS[type_name], data.ctypes.data, data.size, input_size, row_count,
                                      ctypes.byref(out))
    if code == HP_ERR_TYPE:
        return None
    assertHipOk(code, "createQuantizedWeightHandle")
    return HipQuantizedWeightHandle(out.value, type_name, int(data.size), row_count, input_size)


def releaseHipQuantizedWeightHandle(handle: HipQuantizedWeightHandle) -> None:
    """releaseWasmQuantizedWeightHandle (576-584): unknown handles are ignored."""
    if handle.released:
        return
    lib().hp_hip_weight_release(handle.handle)
    handle.released = True


def hipResidentWeightStats() -> dict:
    """wasmResidentWeightStats (586-591) plus runner counters."""
    s = HipStats()
    assertHipOk(lib().hp_hip_stats(ctypes.byref(s)), "residentWeightStats")
    return {
        "instanceCount": 1 if s.device >= 0 else 0,
        "residentBytes": int(s.resident_bytes),
        "handleCount": int(s.handle_count),
        "scratchBytes": int(s.scratch_bytes),
        "matmulCalls": int(s.matmul_calls),
        "kernelLaunches": int(s.kernel_launches),
        "device": int(s.device),
        "computeUnits": int(s.compute_units),
    }


def matMulQuantizedHipResident(handle: HipQuantizedWeightHandle, input_columns, input_size: int, row_count: int,
                               column_count: int) -> np.ndarray:
    """matMulQuantizedWasmResident (593-646): returns [columnCount * rowCount] f32."""
    if handle.released:
        raise RuntimeError(f"Resident quantized matmul handle {handle.handle} is not available")
    if handle.inputSize != input_size or handle.rowCount != row_count:
        raise ValueError(f"Resident quantized matmul handle shape mismatch: {handle.inputSize}x{handle.rowCount}")
    x = _f32(input_columns)
    if x.size != input_size * column_count:
        raise ValueError(f"Resident quantized matmul input shape mismatch: {x.size}")
    out = np.empty(row_count * column_count, dtype=np.float32)
    code = lib().hp_hip_matmul(handle.handle, x.ctypes.data, x.size, input_size, row_count, column_count,
                               out.ctypes.data, out.size)
    assertHipOk(code, "matMulQuantizedResident")
    return out


def matMulQuantizedHipResidentMulti(handles: Sequence[HipQuantizedWeightHandle], input_columns, input_size: int,
                                    column_count: int) -> Optional[list]:
    """matMulQuantizedWasmResidentMulti (648-749): 2..4 handles, one shared Q8_K."""
    if len(handles) < 2 or len(handles) > 4:
        return None
    x = _f32(input_columns)
    if x.size != input_size * column_count:
        raise ValueError(f"Resident quantized multi matmul input shape mismatch: {x.size}")
    for h in handles:
        if h.inputSize != input_size:
            raise ValueError(f"Resident quantized multi matmul handle shape mismatch: {h.inputSize}")
        if h.released:
            raise RuntimeError(f"Resident quantized multi matmul handle {h.handle} is not available")
    n = len(handles)
    outs = [np.empty(h.rowCount * column_count, dtype=np.float32) for h in handles]
    hs = (_u64 * n)(*[h.handle for h in handles])
    optr = (ctypes.c_void_p * n)(*[o.ctypes.data for o in outs])
    olen = (_sz * n)(*[o.size for o in outs])
    code = lib().hp_hip_matmul_multi(n, hs, x.ctypes.data, x.size, input_size, column_count, optr, olen)
    assertHipOk(code, "MatMulQuantizedResidentMulti")
    return outs


def dequantizeHipResident(handle: HipQuantizedWeightHandle, row_start: int, row_count: int) -> np.ndarray:
    """Dequantised rows [row_start, row_start+row_count) as [row_count][inputSize] f32."""
    out = np.empty((row_count, handle.inputSize), dtype=np.float32)
    code = lib().hp_hip_dequantize(handle.handle, row_start, row_count, out.ctypes.data, out.size)
    assertHipOk(code, "dequantize")
    return out


def quantizeQ8KHip(input_columns, input_size: int, column_count: int):
    """Q8_K of each column as the matvec prologue computes it: (qs, d, bsums32)."""
    x = _f32(input_columns)
    qs = np.empty((column_count, input_size), dtype=np.int8)
    d = np.empty((column_count, input_size // 256), dtype=np.float32)
    bs = np.empty((column_count, input_size // 32), dtype=np.int16)
    code = lib().hp_hip_quantize_q8_k(x.ctypes.data, x.size, input_size, column_count, qs.ctypes.data,
                                      d.ctypes.data, bs.ctypes.data)
    assertHipOk(code, "quantizeQ8K")
    return qs, d, bs


def _topk_result(ids: np.ndarray, vals: np.ndarray, n: int, k: int) -> list:
    count = min(n, k)
    return [[{"id": int(i), "value": float(v)} for i, v in zip(ids[r, :count], vals[r, :count])]
            for r in range(ids.shape[0])]


def topKHip(values, k: int, softcap: float = 0.0) -> list:
    """topK (runtime.ts:514-527) of each row of ``values`` ([rows][n] or [n]) on
    the GPU: per row a list of {id, value}, best first, ties to the lower id."""
    v = np.ascontiguousarray(np.atleast_2d(values), dtype=np.float32)
    rows, n = v.shape
    ids = np.empty((rows, k), dtype=np.uint32)
    vals = np.empty((rows, k), dtype=np.float32)
    code = lib().hp_hip_topk(v.ctypes.data, rows, n, k, float(softcap), ids.ctypes.data, vals.ctypes.data,
                             ids.size)
    assertHipOk(code, "topK")
    return _topk_result(ids, vals, n, k)


def matMulQuantizedHipResidentTopK(handle: HipQuantizedWeightHandle, input_columns, input_size: int,
                                   column_count: int, top_k: int, softcap: float = 0.0) -> list:
    """forwardOutput (layers.ts:381-416) for a resident head: logits stay in HBM,
    optional softcap, topK per column; only the candidates come back."""
    if handle.released:
        raise RuntimeError(f"Resident quantized matmul handle {handle.handle} is not available")
    x = _f32(input_columns)
    if handle.inputSize != input_size or x.size != input_size * column_count:
        raise ValueError(f"Resident quantized matmul input shape mismatch: {x.size}")
    ids = np.empty((column_count, top_k), dtype=np.uint32)
    vals = np.empty((column_count, top_k), dtype=np.float32)
    code = lib().hp_hip_matmul_topk(handle.handle, x.ctypes.data, x.size, input_size, column_count, top_k,
                                    float(softcap), ids.ctypes.data, vals.ctypes.data, ids.size)
    assertHipOk(code, "matMulQuantizedResidentTopK")
    return _topk_result(ids, vals, handle.rowCount, top_k)


def matMulGegluHipResident(gate: HipQuantizedWeightHandle, up: HipQuantizedWeightHandle, input_columns,
                           input_size: int, column_count: int) -> np.ndarray:
    """forwardFfn's gate/up batch + GeGLU (layers.ts:432-456) on the GPU:
    fround(gelu(gate . x) * (up . x)), [column_count][rows]; one launch for a
    single column of large projections."""
    for h in (gate, up):
        if h.released:
            raise RuntimeError(f"Resident quantized matmul handle {h.handle} is not available")
    x = _f32(input_columns)
    if gate.inputSize != input_size or up.inputSize != input_size or x.size != input_size * column_count:
        raise ValueError(f"Resident quantized matmul input shape mismatch: {x.size}")
    if gate.rowCount != up.rowCount:
        raise ValueError("gate and up row counts differ")
    out = np.empty(gate.rowCount * column_count, dtype=np.float32)
    code = lib().hp_hip_matmul_geglu(gate.handle, up.handle, x.ctypes.data, x.size, input_size, column_count,
                                     out.ctypes.data, out.size)
    assertHipOk(code, "matMulGeglu")
    return out


def matmul_geglu_device(gate: int, up: int, d_input: int, input_size: int, column_count: int, d_output: int,
                        rows: int, stream: int = 0) -> None:
    """Device-pointer gate/up + GeGLU (asynchronous on `stream`)."""
    assertHipOk(lib().hp_hip_matmul_geglu_device(gate, up, d_input, input_size * column_count, input_size,
                                                 column_count, d_output, rows * column_count, stream or None),
                "matMulGegluDevice")


def gegluHip(gate, up) -> np.ndarray:
    """GeGLU (layers.ts:450-456): fround(gelu(gate) * up), elementwise."""
    g = _f32(gate)
    u = _f32(up)
    if g.size != u.size:
        raise ValueError(f"GeGLU shape mismatch: {g.size} vs {u.size}")
    out = np.empty_like(g)
    assertHipOk(lib().hp_hip_geglu(g.ctypes.data, u.ctypes.data, g.size, out.ctypes.data), "geglu")
    return out.reshape(np.shape(gate))


# ---- device-pointer entry points (inputs/outputs already in HBM) -----------------
def matmul_multi_device(handles: Sequence[int], d_input: int, input_size: int, column_count: int,
                        d_outputs: Sequence[int], output_lens: Sequence[int], stream: int = 0) -> None:
    n = len(handles)
    hs = (_u64 * n)(*handles)
    optr = (ctypes.c_void_p * n)(*d_outputs)
    olen = (_sz * n)(*output_lens)
    code = lib().hp_hip_matmul_multi_device(n, hs, d_input, input_size * column_count, input_size, column_count,
                                            optr, olen, stream or None)
    assertHipOk(code, "matmulMultiDevice")


MATVEC_AUTO, MATVEC_VALU, MATVEC_MFMA, MATVEC_HALF, MATVEC_PREFILL, MATVEC_PREFILL_FAST, MATVEC_WIDE = \
    0, 1, 2, 3, 4, 5, 6
MATVEC_WIDE_WHOLE, MATVEC_WIDE_HALF = 7, 8


def setMatvecKernel(which: int) -> None:
    """Select the matvec kernel (0 automatic, 1 vector ALU, 2 matrix cores,
    3 half-split vector ALU, 4 bit-exact prefill, 5 fast prefill, 6 wide,
    7 / 8 wide with whole / half row-blocks per thread).  1-4 and 6-8 are
    bit-exact; 5 (and the automatic choice from 64 columns) agrees within
    the 1e-4 relative tolerance of projections.  No counterpart in the
    reference."""
    assertHipOk(lib().hp_hip_set_matvec_kernel(int(which)), "setMatvecKernel")


def setInputImages(enable: bool) -> None:
    """Test switch: pre-quantised input images inside draft steps (default on)."""
    assertHipOk(lib().hp_hip_set_input_images(1 if enable else 0), "setInputImages")


def setPrefillFolds(enable: bool) -> None:
    """Test switch: a prefill chunk's launch folds (tiles written by their
    producers, block-range sums added by their consumers, f16 queries);
    default on."""
    assertHipOk(lib().hp_hip_set_prefill_folds(1 if enable else 0), "setPrefillFolds")


def setWeightLayouts(both: bool) -> None:
    """Resident layouts of weights uploaded from now on: both (default) keeps
    the vector-ALU tiles and the matrix-core segments; one layout keeps the
    tiles only (the GGUF byte count), and the matrix-core kernels read them."""
    assertHipOk(lib().hp_hip_set_weight_layouts(1 if both else 0), "setWeightLayouts")


def setDecodeFused(enable: bool) -> None:
    """One-token decode steps as the persistent launch where it applies, or
    always as the launch sequence (the default, and the faster of the two).
    No counterpart in the reference; both give identical bits."""
    assertHipOk(lib().hp_hip_set_decode_fused(1 if enable else 0), "setDecodeFused")


def setFusedWaitLimit(ticks: int) -> None:
    """Bound of one stage wait of the persistent decode step, in 10 ns ticks
    (0: the default, one second).  A test hook: a tiny bound makes a step
    stop at its first wait and report it through decodeFusedStatus."""
    assertHipOk(lib().hp_hip_set_fused_wait_limit(int(ticks)), "setFusedWaitLimit")


def decodeFusedStatus(stream: int = 0) -> int:
    """Waits for `stream` and returns the status of the persistent decode
    steps queued on it (0, or HP_ERR_HIP when one stopped at a wait; the
    status is cleared by reading it)."""
    return int(lib().hp_hip_decode_fused_status(stream or None))


def setFusedTrace(d_stamps: int, length: int) -> None:
    """Stage timeline of the persistent decode step into a device buffer of
    uint64 stamps (0 turns it off); layout in include/hp_hip.h."""
    assertHipOk(lib().hp_hip_set_fused_trace(d_stamps or None, int(length)), "setFusedTrace")


def releaseStreamScratch(stream: int) -> None:
    """Frees the device scratch kept for `stream` (its work done, no graph
    captured on it replayed later); no counterpart in the reference."""
    assertHipOk(lib().hp_hip_release_stream_scratch(stream or None), "releaseStreamScratch")


def emptyLaunches(count: int, stream: int = 0) -> None:
    """count launches of an empty kernel on stream: the floor of a launch or
    graph node (a measurement hook; no counterpart in the reference)."""
    assertHipOk(lib().hp_hip_empty_launches(int(count), stream or None), "emptyLaunches")


def profile(enable: bool) -> None:
    assertHipOk(lib().hp_hip_profile(1 if enable else 0), "profile")


def profile_read(kernel: int) -> tuple[float, int]:
    ms = ctypes.c_double(0)
    n = _u64(0)
    assertHipOk(lib().hp_hip_profile_read(kernel, ctypes.byref(ms), ctypes.byref(n)), "profileRead")
    return ms.value, n.value


def synchronize() -> None:
    assertHipOk(lib().hp_hip_synchronize(), "synchronize")


def shutdown() -> None:
    assertHipOk(lib().hp_hip_shutdown(), "shutdown")


# ---- sampling (generation.ts:40-165) -----------------------------------------

DEFAULT_SAMPLING_SEED = 0x48454C49
DEFAULT_GENERATION_CONFIG = {"doSample": True, "temperature": 1.0, "topP": 0.95, "topK": 64}


def resolveGenerationSamplingOptions(doSample=None, temperature=None, topP=None, topK=None, seed=None) -> dict:
    """resolveGenerationSamplingOptions (generation.ts:40-76): defaults,
    validation (same messages), floor(topK), seed >>> 0, logitsTopK."""
    import math

    d = DEFAULT_GENERATION_CONFIG["doSample"] if doSample is None else doSample
    t = DEFAULT_GENERATION_CONFIG["temperature"] if temperature is None else temperature
    p = DEFAULT_GENERATION_CONFIG["topP"] if topP is None else topP
    k = DEFAULT_GENERATION_CONFIG["topK"] if topK is None else topK
    s = DEFAULT_SAMPLING_SEED if seed is None else seed
    if not math.isfinite(t) or t < 0:
        raise ValueError("temperature must be a finite number greater than or equal to 0.")
    if not math.isfinite(p) or p <= 0 or p > 1:
        raise ValueError("topP must be a finite number in the range (0, 1].")
    if not math.isfinite(k) or k < 1:
        raise ValueError("topK must be a positive finite number.")
    if not math.isfinite(s):
        raise ValueError("seed must be a finite number.")
    k = max(1, math.floor(k))
    greedy = d is False or t == 0
    return {"doSample": d, "temperature": float(t), "topP": float(p), "topK": k,
            "seed": math.floor(s) & 0xFFFFFFFF, "logitsTopK": 1 if greedy else k}


class HipSamplingState:
    """The generator of createDeterministicRng (generation.ts:78-87) as a
    32-bit state that the GPU advances; seeded like the reference."""

    def __init__(self, seed=DEFAULT_SAMPLING_SEED):
        import math

        self.state = ctypes.c_uint32(math.floor(seed) & 0xFFFFFFFF)


def _sampling_struct(o: dict) -> HipSampling:
    return HipSampling(0 if o["doSample"] is False else 1, min(int(o["topK"]), 2 ** 31 - 1), float(o["temperature"]),
                       float(o["topP"]))


def matMulQuantizedHipResidentTopKSample(handle: HipQuantizedWeightHandle, input_columns, input_size: int,
                                         column_count: int, sampling: dict, state: HipSamplingState,
                                         softcap: float = 0.0, top_k: Optional[int] = None) -> list:
    """forwardOutput + sampleNextToken per column on the GPU: the head, its
    top-k (k = sampling["logitsTopK"] unless given) and the sampled token.
    Returns per column {"token", "distribution": [{id, value, probability}]};
    ``state`` advances once per sampled column."""
    if handle.released:
        raise RuntimeError(f"Resident quantized matmul handle {handle.handle} is not available")
    x = _f32(input_columns)
    if handle.inputSize != input_size or x.size != input_size * column_count:
        raise ValueError(f"Resident quantized matmul input shape mismatch: {x.size}")
    k = int(sampling["logitsTopK"] if top_k is None else top_k)
    ids = np.empty((column_count, k), dtype=np.uint32)
    vals = np.empty((column_count, k), dtype=np.float32)
    probs = np.empty((column_count, k), dtype=np.float64)
    tokens = np.empty(column_count, dtype=np.int32)
    kept = np.empty(column_count, dtype=np.int32)
    opts = _sampling_struct(sampling)
    code = lib().hp_hip_matmul_topk_sample(handle.handle, x.ctypes.data, x.size, input_size, column_count, k,
                                           float(softcap), ctypes.byref(opts), ctypes.byref(state.state),
                                           tokens.ctypes.data, ids.ctypes.data, vals.ctypes.data, probs.ctypes.data,
                                           kept.ctypes.data, ids.size)
    assertHipOk(code, "matMulQuantizedResidentTopKSample")
    out = []
    for c in range(column_count):
        n = int(kept[c])
        out.append({"token": int(tokens[c]),
                    "distribution": [{"id": int(ids[c, i]), "value": float(vals[c, i]),
                                      "probability": float(probs[c, i])} for i in range(n)]})
    return out


def sample_device(d_ids: int, d_values: int, column_count: int, k: int, count: int, sampling: dict, d_rng_state: int,
                  d_tokens: int, d_probabilities: int, d_kept: int, stream: int = 0) -> None:
    """hp_hip_sample_device over device pointers (asynchronous on ``stream``)."""
    opts = _sampling_struct(sampling)
    code = lib().hp_hip_sample_device(d_ids, d_values, column_count, k, count, ctypes.byref(opts), d_rng_state,
                                      d_tokens, d_probabilities, d_kept, stream or None)
    assertHipOk(code, "sample")


# ---- decoder layer (device pointers; asynchronous on ``stream``) ----------

def attention_config(head_count: int, head_count_kv: int, capacity: int, *, head_dim: int = 256,
                     rope_dims: int = 256, rope_freq_base: float = 10000.0, d_rope_freq_factors: int = 0,
                     sliding_window: int = 0, epsilon: float = 1e-6) -> HipAttentionConfig:
    """hp_hip_attention_config_t from the manifest's attention fields."""
    return HipAttentionConfig(head_count, head_count_kv, head_dim, rope_dims, rope_freq_base,
                              d_rope_freq_factors or None, capacity, sliding_window, epsilon)


def rms_norm_device(d_input: int, rows: int, n: int, d_weight: int, epsilon: float, d_output: int,
                    stream: int = 0) -> None:
    """rmsNormRows (d_weight 0: rmsNormRowsNoWeight) on device rows."""
    assertHipOk(lib().hp_hip_rms_norm_device(d_input, rows, n, d_weight or None, epsilon, d_output,
                                             stream or None), "rms_norm")


def residual_norm_device(d_branch: int, rows: int, n: int, d_post_weight: int, d_residual: int, scale: float,
                         d_residual_out: int, d_next_weight: int, d_next_out: int, epsilon: float,
                         stream: int = 0) -> None:
    """Post-norm residual add (times scale), then the next norm (d_next_out 0: none)."""
    assertHipOk(lib().hp_hip_residual_norm_device(d_branch, rows, n, d_post_weight or None, d_residual, scale,
                                                  d_residual_out, d_next_weight or None, d_next_out or None,
                                                  epsilon, stream or None), "residual_norm")


def attention_prep_device(config: HipAttentionConfig, d_q: int, d_k: int, d_v: int, d_q_norm: int, d_k_norm: int,
                          d_position: int, d_q_out: int, d_key_cache: int, d_value_cache: int,
                          stream: int = 0, token_count: int = 1) -> None:
    """q/k head norms + RoPE, v norm, and the KV-cache append of tokens at
    *d_position + t."""
    assertHipOk(lib().hp_hip_attention_prep_device(ctypes.byref(config), token_count, d_q, d_k, d_v or None, d_q_norm,
                                                   d_k_norm, d_position, d_q_out, d_key_cache, d_value_cache,
                                                   stream or None), "attention_prep")


def gqa_attention_device(config: HipAttentionConfig, d_q: int, d_key_cache: int, d_value_cache: int,
                         d_position: int, d_output: int, stream: int = 0, token_count: int = 1) -> None:
    """GQA attention of the tokens at *d_position + t (causal), output f16-rounded."""
    assertHipOk(lib().hp_hip_gqa_attention_device(ctypes.byref(config), token_count, d_q, d_key_cache,
                                                  d_value_cache, d_position, d_output, stream or None),
                "gqa_attention")


def decode_layers_device(layers: Sequence[HipDecodeLayer], d_hidden: int, d_position: int,
                         d_output_norm: int = 0, d_output: int = 0, stream: int = 0, token_count: int = 1) -> None:
    """forwardAttentionLayer for the tokens at *d_position + t through
    ``layers`` (hidden [token][hidden] in place), then the final norm into
    d_output when d_output_norm is given."""
    arr = (HipDecodeLayer * len(layers))(*layers)
    assertHipOk(lib().hp_hip_decode_layers_device(arr, len(layers), token_count, d_hidden, d_position,
                                                  d_output_norm or None, d_output or None, stream or None),
                "decode_layers")
