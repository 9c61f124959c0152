"""GGUF files on the HIP runner: parse (C++ reader in csrc/gguf.hip) and
stream tensors from the file into HBM-resident handles.

Mirrors the engine's reader API where the resident-weight path touches it:

==============================================  ==========================================
reference                                       this module
==============================================  ==========================================
``parseGguf`` (gguf.ts:150-215)                 ``parseGguf`` (same result shape)
``tensorByteLength`` (tensor-reader.ts:268)     ``tensorByteLength``
``GgufTensorReader.getTensor`` /                ``GgufFile.getTensor`` / ``readTensorBytes``
``readTensorBytes`` (tensor-reader.ts:66-118)
``readWasmWeightHandle`` (acceleration.ts:164)  ``GgufHipWeights.handle`` (session cache)
==============================================  ==========================================

plus ``GgufHipWeights.upload`` / ``upload_all``, which load many tensors in
one call through ``hp_hip_weight_upload_gguf`` (file -> pinned chunks ->
HBM, with parallel readers).  ``write_gguf`` writes GGUF v3 files (the
synthetic model files of the tests and the bench).
"""
from __future__ import annotations

import ctypes
import os
import struct
from pathlib import Path
from typing import Iterable, Optional, Sequence

import numpy as np

from . import hip_kernels as H

GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32 = 0, 1, 2, 3, 4, 5
GGUF_FLOAT32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = 6, 7, 8, 9, 10, 11, 12
HP_ERR_FORMAT, HP_ERR_IO = 21, 22

GGML_TYPE_IDS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_XS": 23,
                 "I32": 26, "BF16": 30}
_TYPE_NAMES = {0: "uint8", 1: "int8", 2: "uint16", 3: "int16", 4: "uint32", 5: "int32", 6: "float32", 7: "bool",
               8: "string", 9: "array", 10: "uint64", 11: "int64", 12: "float64"}
_INTEGER_TYPES = (GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_UINT64, GGUF_INT64)


class GgufError(ValueError):
    """A malformed GGUF file (the TS parser's thrown Error)."""


# ---------------------------------------------------------------- ctypes ----

class _Value(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("number", ctypes.c_double), ("string", ctypes.c_void_p),
                ("string_length", ctypes.c_uint64), ("element_type", ctypes.c_int32), ("length", ctypes.c_uint64),
                ("sample_count", ctypes.c_uint64), ("truncated", ctypes.c_int32), ("node", ctypes.c_uint64)]


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_void_p), ("name_length", ctypes.c_uint64), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.POINTER(ctypes.c_uint64)), ("type_id", ctypes.c_uint32), ("offset", ctypes.c_uint64),
                ("data_offset", ctypes.c_uint64), ("byte_length", ctypes.c_uint64),
                ("storage_known", ctypes.c_int32)]


_declared = False


def _lib() -> ctypes.CDLL:
    global _declared
    L = H.lib()
    if _declared:
        return L
    u64, i32, vp, sz = ctypes.c_uint64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t
    cpp = ctypes.POINTER(ctypes.c_char_p)
    L.hp_gguf_open.argtypes = [ctypes.c_char_p, u64, cpp, sz, ctypes.POINTER(vp)]
    L.hp_gguf_open_memory.argtypes = [vp, sz, u64, cpp, sz, ctypes.POINTER(vp)]
    L.hp_gguf_close.argtypes = [vp]
    L.hp_gguf_close.restype = None
    L.hp_gguf_last_error.argtypes = []
    L.hp_gguf_last_error.restype = ctypes.c_char_p
    L.hp_gguf_header.argtypes = [vp, ctypes.POINTER(ctypes.c_uint32)] + [ctypes.POINTER(u64)] * 5
    L.hp_gguf_metadata_count.argtypes = [vp]
    L.hp_gguf_metadata_count.restype = u64
    L.hp_gguf_metadata_entry.argtypes = [vp, u64, ctypes.POINTER(vp), ctypes.POINTER(u64), ctypes.POINTER(_Value)]
    L.hp_gguf_metadata_find.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(_Value)]
    L.hp_gguf_array_element.argtypes = [vp, u64, u64, ctypes.POINTER(_Value)]
    L.hp_gguf_tensor_info.argtypes = [vp, u64, ctypes.POINTER(_Tensor)]
    L.hp_gguf_find_tensor.argtypes = [vp, ctypes.c_char_p]
    L.hp_gguf_find_tensor.restype = ctypes.c_int64
    L.hp_gguf_type_name.argtypes = [ctypes.c_uint32]
    L.hp_gguf_type_name.restype = ctypes.c_char_p
    L.hp_gguf_read.argtypes = [vp, u64, vp, u64]
    L.hp_hip_weight_upload_gguf.argtypes = [vp, sz, ctypes.POINTER(u64), ctypes.POINTER(u64), ctypes.POINTER(i32)]
    for name in ("hp_gguf_open", "hp_gguf_open_memory", "hp_gguf_header", "hp_gguf_metadata_entry",
                 "hp_gguf_metadata_find", "hp_gguf_array_element", "hp_gguf_tensor_info", "hp_gguf_read",
                 "hp_hip_weight_upload_gguf"):
        getattr(L, name).restype = i32
    _declared = True
    return L


def _raise(code: int) -> None:
    msg = _lib().hp_gguf_last_error().decode("utf-8", "replace")
    if code == HP_ERR_FORMAT:
        raise GgufError(msg)
    if code == HP_ERR_IO:
        raise OSError(msg)
    raise RuntimeError(f"GGUF reader failed with code {code} ({msg})")


def _bytes(ptr: int, n: int) -> bytes:
    return ctypes.string_at(ptr, n) if n else b""


class GgufFile:
    """A parsed GGUF file (or buffer) held open by the C++ reader.

    ``metadata`` follows parseGguf's result (gguf.ts:30-37): scalars as
    numbers / bools / strings, arrays as {"type", "length", "sample",
    "truncated"}.  Close it (or use ``with``) to release the file."""

    def __init__(self, source, max_array_sample: int = 16, complete_array_keys: Sequence[str] = ()):
        L = _lib()
        keys = [k.encode() for k in complete_array_keys]
        karr = (ctypes.c_char_p * max(1, len(keys)))(*keys)
        out = ctypes.c_void_p()
        self._buf = None
        if isinstance(source, (bytes, bytearray, memoryview, np.ndarray)):
            self._buf = np.frombuffer(bytes(source), dtype=np.uint8) if not isinstance(source, np.ndarray) \
                else np.ascontiguousarray(source, dtype=np.uint8).reshape(-1)
            code = L.hp_gguf_open_memory(self._buf.ctypes.data if self._buf.size else None, self._buf.size,
                                         max_array_sample, karr, len(keys), ctypes.byref(out))
        else:
            code = L.hp_gguf_open(os.fsencode(source), max_array_sample, karr, len(keys), ctypes.byref(out))
        if code != 0:
            _raise(code)
        self._g = out
        v, tc, mc, ds, al, fs = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64(), \
            ctypes.c_uint64(), ctypes.c_uint64()
        L.hp_gguf_header(self._g, ctypes.byref(v), ctypes.byref(tc), ctypes.byref(mc), ctypes.byref(ds),
                         ctypes.byref(al), ctypes.byref(fs))
        self.version, self.tensorCount, self.metadataCount = v.value, tc.value, mc.value
        self.dataStart, self.alignment, self.fileSize = ds.value, al.value, fs.value
        self.metadata = {}
        val = _Value()
        key, klen = ctypes.c_void_p(), ctypes.c_uint64()
        for i in range(L.hp_gguf_metadata_count(self._g)):
            L.hp_gguf_metadata_entry(self._g, i, ctypes.byref(key), ctypes.byref(klen), ctypes.byref(val))
            self.metadata[_bytes(key.value, klen.value).decode("utf-8", "replace")] = self._value(val)
        self.tensors = [self._tensor(i) for i in range(self.tensorCount)]

    def _value(self, v: _Value):
        if v.type == GGUF_STRING:
            return _bytes(v.string, v.string_length).decode("utf-8", "replace")
        if v.type == GGUF_BOOL:
            return v.number != 0
        if v.type in _INTEGER_TYPES:
            return int(v.number)
        if v.type in (GGUF_FLOAT32, GGUF_FLOAT64):
            return float(v.number)
        sample = []
        child = _Value()
        for j in range(v.sample_count):
            _lib().hp_gguf_array_element(self._g, v.node, j, ctypes.byref(child))
            sample.append(self._value(child))
        return {"type": _TYPE_NAMES.get(v.element_type, "array"), "length": int(v.length), "sample": sample,
                "truncated": bool(v.truncated)}

    def _tensor(self, i: int) -> dict:
        t = _Tensor()
        _lib().hp_gguf_tensor_info(self._g, i, ctypes.byref(t))
        name = _bytes(t.name, t.name_length).decode("utf-8", "replace")
        return {"name": name, "dimensions": [int(t.dims[d]) for d in range(t.n_dims)],
                "type": _lib().hp_gguf_type_name(t.type_id).decode(), "typeId": int(t.type_id),
                "offset": int(t.offset), "dataOffset": int(t.data_offset),
                "byteLength": int(t.byte_length) if t.storage_known else None, "index": i}

    # -- GgufTensorReader-like access ------------------------------------
    def getTensor(self, name: str) -> dict:
        idx = _lib().hp_gguf_find_tensor(self._g, name.encode())
        if idx < 0:
            raise KeyError(f"Unknown tensor: {name}")
        return self.tensors[idx]

    def readTensorBytes(self, name: str) -> np.ndarray:
        t = self.getTensor(name)
        n = tensorByteLength(t)
        out = np.empty(n, dtype=np.uint8)
        code = _lib().hp_gguf_read(self._g, t["dataOffset"], out.ctypes.data, n)
        if code != 0:
            _raise(code)
        return out

    def as_dict(self) -> dict:
        """parseGguf's GgufMetadata shape."""
        return {"version": self.version, "tensorCount": self.tensorCount, "metadataCount": self.metadataCount,
                "metadata": self.metadata, "dataStart": self.dataStart,
                "tensors": [{k: t[k] for k in ("name", "dimensions", "type", "typeId", "offset", "dataOffset")}
                            for t in self.tensors]}

    def close(self) -> None:
        if getattr(self, "_g", None):
            _lib().hp_gguf_close(self._g)
            self._g = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def parseGguf(source, maxArraySample: int = 16, completeArrayKeys: Sequence[str] = ()) -> dict:
    """parseGguf (gguf.ts:150-215) of a path or a bytes buffer."""
    with GgufFile(source, maxArraySample, completeArrayKeys) as g:
        return g.as_dict()


def tensorByteLength(tensor: dict) -> int:
    """tensorByteLength (tensor-reader.ts:268-280); raises for an unknown storage type."""
    if tensor.get("byteLength") is None:
        raise GgufError(f"Unsupported tensor storage type or shape: {tensor['type']} {tensor['dimensions']}")
    return tensor["byteLength"]


class GgufHipWeights:
    """Session-scoped cache of HBM-resident weight handles keyed by tensor
    name: readWasmWeightHandle (acceleration.ts:164-201) on the GPU.
    ``handle(name)`` uploads on first use; ``upload(names)`` loads many
    tensors in one streamed call.  Tensors of block types the runner does
    not implement give None (the engine falls back)."""

    def __init__(self, gguf: GgufFile):
        self.gguf = gguf
        self.handles: dict = {}
        self.unsupported: set = set()
        self.hits = 0
        self.misses = 0
        self.bytes = 0

    def upload(self, names: Iterable[str]) -> dict:
        todo = [n for n in dict.fromkeys(names) if n not in self.handles and n not in self.unsupported]
        if todo:
            tensors = [self.gguf.getTensor(n) for n in todo]
            k = len(tensors)
            idx = (ctypes.c_uint64 * k)(*[t["index"] for t in tensors])
            hs = (ctypes.c_uint64 * k)()
            st = (ctypes.c_int32 * k)()
            code = _lib().hp_hip_weight_upload_gguf(self.gguf._g, k, idx, hs, st)
            H.assertHipOk(code, "uploadGgufWeights")
            for t, h, s in zip(tensors, hs, st):
                if s == H.HP_ERR_TYPE:
                    self.unsupported.add(t["name"])
                    continue
                self.handles[t["name"]] = H.HipQuantizedWeightHandle(
                    int(h), t["type"], t["byteLength"], t["dimensions"][1], t["dimensions"][0])
                self.bytes += t["byteLength"]
        return {n: self.handles.get(n) for n in names}

    def upload_all(self) -> dict:
        return self.upload([t["name"] for t in self.gguf.tensors])

    def handle(self, name: str) -> Optional[H.HipQuantizedWeightHandle]:
        if name in self.handles:
            self.hits += 1
            return self.handles[name]
        self.misses += 1
        return self.upload([name])[name]

    def release(self) -> None:
        for h in self.handles.values():
            H.releaseHipQuantizedWeightHandle(h)
        self.handles.clear()


# ---------------------------------------------------------------- writer ----

def _pack_value(type_id: int, value) -> bytes:
    if type_id == GGUF_STRING:
        b = value.encode() if isinstance(value, str) else bytes(value)
        return struct.pack("<Q", len(b)) + b
    if type_id == GGUF_ARRAY:
        elem, items = value
        return struct.pack("<IQ", elem, len(items)) + b"".join(_pack_value(elem, x) for x in items)
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q",
           12: "<d"}[type_id]
    return struct.pack(fmt, int(value) if type_id == GGUF_BOOL else value)


def gguf_header(metadata: Sequence[tuple], tensors: Sequence[tuple], alignment: int = 32,
                version: int = 3) -> tuple:
    """GGUF v3 header bytes for ``metadata`` [(key, type_id, value)] (array
    values as (element_type, items)) and ``tensors`` [(name, dims,
    ggml_type_id, nbytes)].  Tensor data is laid out in order, each start
    aligned.  Returns (header padded to the data start, [data offsets])."""
    out = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(metadata))]
    for key, type_id, value in metadata:
        out += [_pack_value(GGUF_STRING, key), struct.pack("<I", type_id), _pack_value(type_id, value)]
    offsets, at = [], 0
    for name, dims, type_id, nbytes in tensors:
        offsets.append(at)
        out += [_pack_value(GGUF_STRING, name), struct.pack("<I", len(dims)),
                b"".join(struct.pack("<Q", d) for d in dims), struct.pack("<IQ", type_id, at)]
        at += nbytes
        at += -at % alignment
    head = b"".join(out)
    head += b"\0" * (-len(head) % alignment)
    return head, offsets


def write_gguf(path, metadata: Sequence[tuple], tensors: Sequence[tuple], alignment: int = 32) -> Path:
    """Write a GGUF v3 file; ``tensors``: [(name, dims, ggml_type_id, data)]
    with data as bytes or a uint8 array."""
    items = [(n, d, t, np.ascontiguousarray(x, dtype=np.uint8).reshape(-1) if isinstance(x, np.ndarray) else bytes(x))
             for n, d, t, x in tensors]
    return _write(path, metadata, items, [len(x) for _, _, _, x in items], alignment)


def _write(path, metadata, tensors, sizes, alignment) -> Path:
    head, offsets = gguf_header(metadata, [(n, d, t, s) for (n, d, t, _), s in zip(tensors, sizes)], alignment)
    path = Path(path)
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for (_, _, _, data), off, size in zip(tensors, offsets, sizes):
            if off > pos:
                f.write(b"\0" * (off - pos))
                pos = off
            blob = data[1]() if isinstance(data, tuple) else data
            b = np.ascontiguousarray(blob, dtype=np.uint8).reshape(-1) if isinstance(blob, np.ndarray) else blob
            if len(memoryview(b).cast("B")) != size:
                raise ValueError("tensor data length differs from its declared size")
            f.write(b)
            pos += size
    return path


def write_gguf_lazy(path, metadata: Sequence[tuple], tensors: Sequence[tuple], alignment: int = 32) -> Path:
    """write_gguf for [(name, dims, ggml_type_id, nbytes, make_bytes)]: each
    tensor's bytes are made just before they are written."""
    items = [(n, d, t, (s, fn)) for n, d, t, s, fn in tensors]
    return _write(path, metadata, items, [s for _, _, _, s, _ in tensors], alignment)
