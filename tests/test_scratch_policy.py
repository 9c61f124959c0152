"""CPU check of the device-scratch policy of the asynchronous entry points
(heliopause_amd/csrc/hp_scratch.h): per stream, grow-only, no buffer freed
before shutdown (a captured HIP graph may hold it), no growth while a stream
captures.  The policy header is compiled with g++ against a recording
allocator (tests/scratch_policy.cpp); no GPU is involved."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_scratch_policy(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "scratch_policy"
    subprocess.run([cxx, "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'heliopause_amd' / 'csrc'}",
                    str(ROOT / "tests" / "scratch_policy.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "scratch policy ok" in r.stdout
