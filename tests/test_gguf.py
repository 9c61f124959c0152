"""GGUF reader: the C++ reader (csrc/gguf.hip, via heliopause_amd.gguf)
against the oracle's restatement of parseGguf (oracle/gguf.py), and the
oracle itself against the reference's known answers.

Known answers (packages/engine/test/chat.test.ts): "file GGUF tensor reader
uses File.slice ranges" (436-453, bytes from minimalGgufBytes 695-709) and
"file GGUF tensor reader fully parses tokenizer arrays" (455-480, bytes
from tokenizerArrayGgufBytes 711-733).  The byte layouts those builders
produce are written here field by field with this repository's writer.
"""
import struct

import numpy as np
import pytest

from heliopause_amd import gguf as G
from oracle import gguf as OG


def _u32(v):
    return struct.pack("<I", v)


def _u64(v):
    return struct.pack("<Q", v)


def _str(s):
    b = s.encode()
    return _u64(len(b)) + b


def _pad(b, a=32):
    return b + b"\0" * (-len(b) % a)


def minimal_gguf(tensor_bytes: bytes) -> bytes:
    """minimalGgufBytes: v3, 1 tensor "weight" dims [4] F32 offset 0, no metadata."""
    head = b"GGUF" + _u32(3) + _u64(1) + _u64(0) + _str("weight") + _u32(1) + _u64(4) + _u32(0) + _u64(0)
    return _pad(head) + tensor_bytes


def tokenizer_gguf(tokens, merges) -> bytes:
    """tokenizerArrayGgufBytes: two string arrays, no tensors."""
    b = b"GGUF" + _u32(3) + _u64(0) + _u64(2)
    for key, items in (("tokenizer.ggml.tokens", tokens), ("tokenizer.ggml.merges", merges)):
        b += _str(key) + _u32(9) + _u32(8) + _u64(len(items)) + b"".join(_str(x) for x in items)
    return _pad(b)


TOKENIZER_KEYS = ("tokenizer.ggml.tokens", "tokenizer.ggml.merges")  # chat.ts:149-152


@pytest.mark.parametrize("parse", ["oracle", "hip"])
def test_reference_minimal_file(parse, tmp_path):
    tensor = np.array([1, 2, 3, 4], np.float32).tobytes()
    data = minimal_gguf(tensor)
    if parse == "oracle":
        g = OG.parse_gguf(data)
        t = g["tensors"][0]
        got = data[t["dataOffset"]:t["dataOffset"] + OG.tensor_byte_length(t)]
    else:
        path = tmp_path / "m.gguf"
        path.write_bytes(data)
        with G.GgufFile(path) as f:
            g = f.as_dict()
            got = f.readTensorBytes("weight").tobytes()
            t = f.getTensor("weight")
    assert got == tensor                                      # chat.test.ts:451
    assert (g["version"], g["tensorCount"], g["metadataCount"], g["dataStart"]) == (3, 1, 0, 64)
    assert (t["name"], t["dimensions"], t["type"], t["typeId"], t["offset"]) == ("weight", [4], "F32", 0, 0)


@pytest.mark.parametrize("parse", ["oracle", "hip"])
def test_reference_tokenizer_arrays(parse):
    data = tokenizer_gguf(["a", "b", "c"], ["a b", "b c", "c d"])
    run = OG.parse_gguf if parse == "oracle" else G.parseGguf
    md = run(data, 1, TOKENIZER_KEYS)["metadata"]           # chat.test.ts:457-480
    assert md["tokenizer.ggml.tokens"] == {"type": "string", "length": 3, "sample": ["a", "b", "c"],
                                           "truncated": False}
    assert md["tokenizer.ggml.merges"] == {"type": "string", "length": 3, "sample": ["a b", "b c", "c d"],
                                           "truncated": False}
    md = run(data, 1)["metadata"]                            # without the complete keys: sampled
    assert md["tokenizer.ggml.tokens"] == {"type": "string", "length": 3, "sample": ["a"], "truncated": True}


# ---- generated files ---------------------------------------------------------

def _random_value(rng, type_id, depth=0):
    if type_id == G.GGUF_STRING:
        return "".join(chr(c) for c in rng.integers(32, 127, size=int(rng.integers(0, 12)))) + \
            ("é中" if rng.random() < 0.2 else "")
    if type_id == G.GGUF_ARRAY:
        elem = int(rng.choice([0, 1, 2, 3, 4, 5, 6, 7, 8, 10, 11, 12] + ([9] if depth < 2 else [])))
        return elem, [_random_value(rng, elem, depth + 1) for _ in range(int(rng.integers(0, 6)))]
    lo_hi = {0: (0, 255), 1: (-128, 127), 2: (0, 65535), 3: (-32768, 32767), 4: (0, 2 ** 32 - 1),
             5: (-2 ** 31, 2 ** 31 - 1), 10: (0, 2 ** 53 - 1), 11: (-(2 ** 53 - 1), 2 ** 53 - 1)}
    if type_id in lo_hi:
        lo, hi = lo_hi[type_id]
        return int(rng.choice([lo, hi, int(rng.integers(lo // 2, hi // 2 + 1, dtype=np.int64))]))
    if type_id == G.GGUF_BOOL:
        return bool(rng.integers(0, 2))
    if type_id == G.GGUF_FLOAT32:
        return float(np.float32(rng.standard_normal() * 100))
    return float(rng.standard_normal() * 1e10)


def _expected_value(type_id, value, max_sample):
    """What parseGguf returns for a value written by the writer (independent
    of both parsers): scalars as written, arrays sampled."""
    if type_id != G.GGUF_ARRAY:
        return value
    elem, items = value
    keep = min(len(items), max_sample)
    return {"type": OG.METADATA_TYPE_NAMES[elem], "length": len(items),
            "sample": [_expected_value(elem, x, max_sample) for x in items[:keep]], "truncated": len(items) > keep}


def random_file(seed):
    rng = np.random.default_rng(seed)
    md = []
    for i in range(int(rng.integers(0, 10))):
        t = int(rng.choice([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12]))
        key = f"k.{int(rng.integers(0, 6))}" if rng.random() < 0.3 else f"key.{i}"   # some repeats
        md.append((key, t, _random_value(rng, t)))
    alignment = int(rng.choice([1, 8, 32, 64, 4096]))
    if rng.random() < 0.5:
        md.append(("general.alignment", G.GGUF_UINT32, alignment))
    else:
        alignment = 32
    tensors = []
    for i in range(int(rng.integers(0, 5))):
        typ = str(rng.choice(["Q4_K", "Q6_K", "F32", "Q8_0"]))
        block = 256 if typ in ("Q4_K", "Q6_K") else (32 if typ == "Q8_0" else 1)
        dims = [block * int(rng.integers(1, 3)), int(rng.integers(1, 4))]
        nbytes = OG.tensor_byte_length({"name": "", "dimensions": dims, "type": typ})
        name = "dup" if rng.random() < 0.2 else f"blk.{i}.w"
        tensors.append((name, dims, G.GGML_TYPE_IDS[typ], rng.integers(0, 256, nbytes, dtype=np.uint8)))
    head, offsets = G.gguf_header(md, [(n, d, t, len(x)) for n, d, t, x in tensors], alignment)
    data = bytearray(head)
    for (_, _, _, x), off in zip(tensors, offsets):
        data += b"\0" * (len(head) + off - len(data))
        data += x.tobytes()
    return bytes(data), md, tensors, alignment


@pytest.mark.parametrize("seed", range(40))
def test_random_files_match_oracle_and_writer(seed):
    data, md, tensors, alignment = random_file(seed)
    max_sample = [0, 1, 3, 16][seed % 4]
    ref = OG.parse_gguf(data, max_sample)
    got = G.parseGguf(data, max_sample)
    assert got == ref
    # the oracle against what the writer wrote
    expect = {}
    for key, t, v in md:
        expect[key] = _expected_value(t, v, max_sample)
    assert ref["metadata"] == expect and list(ref["metadata"]) == list(expect)
    assert [t["name"] for t in ref["tensors"]] == [t[0] for t in tensors]
    assert ref["dataStart"] % alignment == 0
    for t, (_, _, _, x) in zip(ref["tensors"], tensors):
        assert data[t["dataOffset"]:t["dataOffset"] + OG.tensor_byte_length(t)] == x.tobytes()
    with G.GgufFile(data) as f:
        for t in tensors:                       # duplicate names resolve to the last, like a Map
            last = max(i for i, u in enumerate(tensors) if u[0] == t[0])
            assert f.getTensor(t[0])["index"] == last
            assert f.readTensorBytes(t[0]).tobytes() == tensors[last][3].tobytes()


def _outcome(fn, data, *args):
    try:
        return ("ok", fn(data, *args))
    except (OG.GgufError, G.GgufError) as e:
        # the C ABI reports errors as C strings: a NUL byte inside a name ends them
        return ("error", str(e).split("\0")[0])


@pytest.mark.parametrize("seed", [1, 7, 12])
def test_every_truncation_matches(seed):
    data, *_ = random_file(seed)
    for cut in range(0, min(len(data), 700)):
        assert _outcome(G.parseGguf, data[:cut], 3) == _outcome(OG.parse_gguf, data[:cut], 3), cut


def test_mutations_match():
    """Byte flips in the header of valid files: both readers reach the same
    result or the same error message (and the C++ reader never crashes)."""
    rng = np.random.default_rng(99)
    for seed in range(12):
        data, *_ = random_file(100 + seed)
        head_len = OG.parse_gguf(data)["dataStart"]
        for _ in range(40):
            b = bytearray(data)
            for _ in range(int(rng.integers(1, 4))):
                b[int(rng.integers(0, max(1, head_len)))] = int(rng.integers(0, 256))
            b = bytes(b)
            assert _outcome(G.parseGguf, b, 4) == _outcome(OG.parse_gguf, b, 4)


@pytest.mark.parametrize("case,message", [
    (b"GGUX" + _u32(3) + _u64(0) + _u64(0), "Invalid GGUF magic: expected GGUF, got GGUX"),
    (b"GGUF" + _u32(3) + _u64(2 ** 53) + _u64(0), "tensor count exceeds JavaScript safe integer range: 9007199254740992"),
    (b"GGUF" + _u32(3) + _u64(0) + _u64(1) + _str("x") + _u32(13), "Unsupported GGUF metadata type id: 13"),
    (b"GGUF" + _u32(3) + _u64(0) + _u64(1) + _str("x") + _u32(10) + _u64(2 ** 63),
     "uint64 metadata value exceeds JavaScript safe integer range: 9223372036854775808"),
    (b"GGUF" + _u32(3) + _u64(0) + _u64(1) + _str("x") + _u32(11) + struct.pack("<q", -(2 ** 53)),
     "int64 metadata value exceeds JavaScript safe integer range: -9007199254740992"),
    (b"GGUF" + _u32(3) + _u64(1) + _u64(0) + _str("t") + _u32(1) + _u64(2 ** 60),
     "dimension for t exceeds JavaScript safe integer range: 1152921504606846976"),
    # a skipped string longer than the file: the skip passes, the next read is past the end
    (b"GGUF" + _u32(3) + _u64(0) + _u64(2) + _str("a") + _u32(9) + _u32(8) + _u64(2) + _str("s") + _u64(1000)
     + _str("b"), "Unexpected EOF at offset 1066"),    # 24 + 9 + 4 + 4 + 8 + 9 + 8 + 1000
    (b"GGUF" + _u32(3) + _u64(0) + _u64(1) + _str("general.alignment") + _u32(4) + _u32(0),
     "general.alignment must be a positive integer"),
])
def test_errors_match(case, message):
    assert _outcome(OG.parse_gguf, case, 1) == ("error", message)
    assert _outcome(G.parseGguf, case, 1) == ("error", message)


def test_alignment_value_kinds():
    """general.alignment counts only when it is a number (getMetadataNumber):
    a string or bool value leaves the default 32."""
    for typ, val, expect in ((G.GGUF_UINT64, 128, 128), (G.GGUF_FLOAT32, 16.0, 16), (G.GGUF_STRING, "64", 32),
                             (G.GGUF_BOOL, True, 32), (G.GGUF_UINT8, 1, 1)):
        head, _ = G.gguf_header([("general.alignment", typ, val)], [("t", [4], 0, 16)], 1)
        data = head + b"\0" * (-len(head) % 256) + bytes(16)
        ref = OG.parse_gguf(data)
        assert ref["dataStart"] % expect == 0
        assert G.parseGguf(data) == ref


def test_tensor_byte_length_table():
    """ggmlTypeStorage (tensor-reader.ts:282-293): known types give
    elements / block * size; unknown types and ragged counts have none."""
    cases = [("F32", [3, 5], 60), ("F16", [7], 14), ("BF16", [2, 2], 8), ("Q4_0", [64], 36), ("Q8_0", [32, 2], 68),
             ("Q4_K", [2560, 2048], 2560 * 2048 // 256 * 144), ("Q5_K", [256], 176), ("Q6_K", [512, 3], 1260),
             ("IQ4_XS", [256], 136), ("I32", [9], 36)]
    md, ts = [], []
    for name, dims, _ in cases:
        ts.append((name, dims, G.GGML_TYPE_IDS[name], 0))
    ts.append(("ragged", [100], G.GGML_TYPE_IDS["Q4_K"], 0))
    ts.append(("q3k", [256], 11, 0))
    head, _ = G.gguf_header(md, ts)
    with G.GgufFile(head) as f:
        for (name, dims, nbytes) in cases:
            assert G.tensorByteLength(f.getTensor(name)) == nbytes
            assert OG.tensor_byte_length(OG.parse_gguf(head)["tensors"][[c[0] for c in cases].index(name)]) == nbytes
        for name in ("ragged", "q3k"):
            with pytest.raises(G.GgufError):
                G.tensorByteLength(f.getTensor(name))
        assert f.getTensor("q3k")["type"] == "Q3_K"
    with pytest.raises(OG.GgufError, match="not divisible by block size 256"):
        OG.tensor_byte_length({"name": "ragged", "dimensions": [100], "type": "Q4_K"})


def test_unknown_type_names_and_missing_tensor():
    head, _ = G.gguf_header([], [("x", [1], 31, 0), ("y", [1], 41, 0)])
    g = G.parseGguf(head)
    assert [t["type"] for t in g["tensors"]] == ["UNKNOWN_31", "Q1_0"] == \
        [t["type"] for t in OG.parse_gguf(head)["tensors"]]
    with G.GgufFile(head) as f, pytest.raises(KeyError, match="Unknown tensor: z"):
        f.getTensor("z")


def test_open_errors(tmp_path):
    with pytest.raises(OSError):
        G.GgufFile(tmp_path / "missing.gguf")
    assert _outcome(G.parseGguf, b"", 1) == ("error", "Unexpected EOF at offset 0")
