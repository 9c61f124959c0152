"""Pure-Python restatement of the engine's GGUF reader (the oracle for the
C++ reader in heliopause_amd/csrc/gguf.hip).

TEST INFRASTRUCTURE ONLY: only tests/ and bench.py's cpu_baseline leg may
import this module; the product path never does.

Follows, function by function:
  parse_gguf          parseGguf                 packages/engine/src/gguf.ts:150-215
  _read_value         readMetadataValue         gguf.ts:265-300
  _read_array         readArraySummary          gguf.ts:302-326
  _skip_value         skipMetadataValue         gguf.ts:328-365
  _align              alignOffset               gguf.ts:367-370
  _safe               bigintToSafeNumber        gguf.ts:372-378
  Cursor              GgufCursor                gguf.ts:380-462
  METADATA_TYPE_NAMES metadataTypeNames         gguf.ts:97-111
  tensor_byte_length  tensorByteLength          packages/engine/src/tensor-reader.ts:268-280
  GGML_TYPE_STORAGE   ggmlTypeStorage           tensor-reader.ts:282-293
  GGML_TYPE_NAMES     ggmlTypeNames             gguf.ts:113-148
Values come back as the TS parser builds them: numbers (int/float), bools,
strings (UTF-8 decoded with replacement, as TextDecoder does) and array
summaries {"type", "length", "sample", "truncated"}.  Metadata is a dict in
first-insertion order with the last value of a repeated key, like a JS
object.  Errors raise GgufError with the TS message.
"""
from __future__ import annotations

import math
import struct

MAX_SAFE = 2 ** 53 - 1
DEFAULT_ALIGNMENT = 32

METADATA_TYPE_NAMES = {
    0: "uint8", 1: "int8", 2: "uint16", 3: "int16", 4: "uint32", 5: "int32", 6: "float32",
    7: "bool", 8: "string", 9: "array", 10: "uint64", 11: "int64", 12: "float64",
}

GGML_TYPE_NAMES = {
    0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1", 10: "Q2_K",
    11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS",
    19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS", 24: "I8", 25: "I16", 26: "I32",
    27: "I64", 28: "F64", 29: "IQ1_M", 30: "BF16", 34: "TQ1_0", 35: "TQ2_0", 39: "MXFP4", 40: "NVFP4",
    41: "Q1_0",
}

GGML_TYPE_STORAGE = {  # name -> (blockSize, typeSize)
    "F32": (1, 4), "F16": (1, 2), "BF16": (1, 2), "Q4_0": (32, 18), "Q8_0": (32, 34), "Q4_K": (256, 144),
    "Q5_K": (256, 176), "Q6_K": (256, 210), "IQ4_XS": (256, 136), "I32": (1, 4),
}

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 12: "<d"}
_SKIP = {0: 1, 1: 1, 7: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 10: 8, 11: 8, 12: 8}


class GgufError(ValueError):
    pass


class Cursor:
    """GgufCursor: reads at ``offset``; a short read is an EOF error at the
    offset before it; skips move the offset without checking."""

    def __init__(self, data: bytes):
        self.data = data
        self.offset = 0

    def read(self, n: int) -> bytes:
        b = self.data[self.offset:self.offset + n] if self.offset <= len(self.data) else b""
        if len(b) != n:
            raise GgufError(f"Unexpected EOF at offset {self.offset}")
        self.offset += n
        return b

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.read(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = _safe(self.unpack("<Q"), "string length")
        return self.read(n).decode("utf-8", errors="replace")

    def skip(self, n: int) -> None:
        self.offset += n


def _safe(v: int, label: str) -> int:
    if v > MAX_SAFE or v < -MAX_SAFE:
        raise GgufError(f"{label} exceeds JavaScript safe integer range: {v}")
    return v


def _read_value(c: Cursor, type_id: int, max_sample: int):
    if type_id in _SCALAR:
        return c.unpack(_SCALAR[type_id])
    if type_id == 7:
        return c.unpack("<B") != 0
    if type_id == 8:
        return c.string()
    if type_id == 9:
        return _read_array(c, max_sample)
    if type_id == 10:
        return _safe(c.unpack("<Q"), "uint64 metadata value")
    if type_id == 11:
        return _safe(c.unpack("<q"), "int64 metadata value")
    raise GgufError(f"Unsupported GGUF metadata type id: {type_id}")


def _read_array(c: Cursor, max_sample: int) -> dict:
    elem = c.unpack("<I")
    length = _safe(c.unpack("<Q"), "array length")
    keep = min(length, max_sample)
    sample = [_read_value(c, elem, max_sample) for _ in range(keep)]
    _skip_values(c, elem, length - keep)
    return {"type": METADATA_TYPE_NAMES.get(elem, "array"), "length": length, "sample": sample,
            "truncated": length > keep}


def _skip_value(c: Cursor, type_id: int) -> None:
    if type_id in _SKIP:
        c.skip(_SKIP[type_id])
    elif type_id == 8:
        c.skip(_safe(c.unpack("<Q"), "string length"))
    elif type_id == 9:
        elem = c.unpack("<I")
        length = _safe(c.unpack("<Q"), "array length")
        _skip_values(c, elem, length)
    else:
        raise GgufError(f"Unsupported GGUF metadata type id: {type_id}")


def _skip_values(c: Cursor, type_id: int, count: int) -> None:
    """``count`` skipMetadataValue calls.  Fixed-size skips read nothing and
    cannot fail, so they are taken at once; strings and arrays read a length
    each and so stop at the end of the data at the latest."""
    if count and type_id in _SKIP:
        c.skip(count * _SKIP[type_id])
        return
    for _ in range(count):
        _skip_value(c, type_id)


def _align(offset: int, alignment: int) -> int:
    rem = offset % alignment
    return offset if rem == 0 else offset + alignment - rem


def parse_gguf(data: bytes, max_array_sample: int = 16, complete_array_keys=()) -> dict:
    c = Cursor(bytes(data))
    complete = set(complete_array_keys)
    magic = c.read(4).decode("latin-1")
    if magic != "GGUF":
        raise GgufError(f"Invalid GGUF magic: expected GGUF, got {magic}")
    version = c.unpack("<I")
    tensor_count = _safe(c.unpack("<Q"), "tensor count")
    metadata_count = _safe(c.unpack("<Q"), "metadata count")
    metadata: dict = {}
    for _ in range(metadata_count):
        key = c.string()
        type_id = c.unpack("<I")
        metadata[key] = _read_value(c, type_id, MAX_SAFE if key in complete else max_array_sample)
    tensors = []
    for _ in range(tensor_count):
        name = c.string()
        nd = c.unpack("<I")
        dims = [_safe(c.unpack("<Q"), f"dimension for {name}") for _ in range(nd)]
        type_id = c.unpack("<I")
        offset = c.unpack("<Q")
        tensors.append({"name": name, "dimensions": dims, "type": GGML_TYPE_NAMES.get(type_id, f"UNKNOWN_{type_id}"),
                        "typeId": type_id, "offset": offset, "dataOffset": 0})
    align_value = metadata.get("general.alignment")
    alignment = align_value if isinstance(align_value, (int, float)) and not isinstance(align_value, bool) \
        else DEFAULT_ALIGNMENT
    if not math.isfinite(alignment) or alignment < 1 or alignment > 2 ** 32 or alignment != int(alignment):
        # BigInt() of a fraction or a non-finite value, or a remainder by 0n,
        # throws a RangeError in the TS parser; a negative or absurdly large
        # alignment has no meaning.  Rejected here.
        raise GgufError("general.alignment must be a positive integer")
    data_start = _align(c.offset, int(alignment))
    for t in tensors:
        t["dataOffset"] = data_start + t["offset"]
    return {"version": version, "tensorCount": tensor_count, "metadataCount": metadata_count,
            "metadata": metadata, "tensors": tensors, "dataStart": data_start}


def tensor_byte_length(tensor: dict) -> int:
    elements = 1
    for d in tensor["dimensions"]:
        elements *= d
    info = GGML_TYPE_STORAGE.get(tensor["type"])
    if info is None:
        raise GgufError(f"Unsupported tensor storage type: {tensor['type']}")
    block, size = info
    if elements % block != 0:
        raise GgufError(f"Tensor {tensor['name']} element count {elements} is not divisible by block size {block}")
    return elements // block * size
