"""The C ABI library loads and exports every entry point include/hp_hip.h
declares; constants match the reference's; the host mirror validates
arguments like wasm-kernels.ts before touching the GPU.  CPU only: no
entry point that reaches the GPU is called here.
"""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hp_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(hp_hip_[a-z_0-9]+)\s*\(", text, re.M)))


def test_library_exports_every_declared_entry_point():
    from heliopause_amd import hip_kernels as H

    L = H.lib()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_one_hip_runtime_in_the_process():
    """With PyTorch installed, the library binds to torch's HIP runtime (one
    libamdhip64 mapped), so torch tensors and streams can be passed in."""
    from heliopause_amd import hip_kernels as H

    H.lib()
    maps = Path("/proc/self/maps").read_text().splitlines()
    runtimes = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes


def test_constants_match_reference():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define (HP_[A-Z0-9_]+) (\d+)", text))
    # lib.rs:7-17
    assert consts["HP_OK"] == "0" and consts["HP_ERR_SHAPE"] == "1"
    assert consts["HP_ERR_HEADS"] == "2" and consts["HP_ERR_TYPE"] == "3"
    assert [consts[f"HP_TYPE_{t}"] for t in ("Q4_K", "Q5_K", "Q6_K", "IQ4_XS", "Q8_0", "Q4_0")] == list("123456")
    from oracle import oracle as O

    assert (O.OK, O.ERR_SHAPE, O.ERR_HEADS, O.ERR_TYPE) == (0, 1, 2, 3)


def test_status_strings():
    from heliopause_amd import hip_kernels as H

    assert H.status_string(0) == "ok"
    assert H.status_string(1) == "shape mismatch"
    assert H.status_string(3) == "unsupported type"
    assert H.status_string(999) == "unknown status"


def test_mirror_validates_before_the_gpu():
    from heliopause_amd import hip_kernels as H

    # quantizedTypeId (wasm-kernels.ts:1908-1923)
    assert [H.quantizedTypeId(t) for t in ("Q4_K", "Q5_K", "Q6_K", "IQ4_XS", "Q8_0", "Q4_0")] == [1, 2, 3, 4, 5, 6]
    assert H.quantizedTypeId("F16") is None
    w = np.zeros(144, np.uint8)
    assert H.createHipQuantizedWeightHandle("Q5_K", w, 256, 1) is None
    with pytest.raises(ValueError):
        H.createHipQuantizedWeightHandle("Q4_K", w, 0, 1)
    with pytest.raises(ValueError):
        H.createHipQuantizedWeightHandle("Q4_K", w, 300, 1)
    h = H.HipQuantizedWeightHandle(1, "Q4_K", 144, 1, 256)
    assert H.matMulQuantizedHipResidentMulti([h], np.zeros(256, np.float32), 256, 1) is None
    with pytest.raises(ValueError):
        H.matMulQuantizedHipResident(h, np.zeros(256, np.float32), 256, 2, 1)
    with pytest.raises(ValueError):
        H.matMulQuantizedHipResident(h, np.zeros(255, np.float32), 256, 1, 1)


def test_assert_ok_messages():
    from heliopause_amd import hip_kernels as H

    H.assertHipOk(0, "x")
    with pytest.raises(ValueError, match="x hip shape mismatch"):
        H.assertHipOk(1, "x")
    with pytest.raises(ValueError, match="head count"):
        H.assertHipOk(2, "x")
    with pytest.raises(TypeError, match="unsupported type"):
        H.assertHipOk(3, "x")
