"""The device kernels round the query to f16 with rs_f16_bits
(heliopause_amd/csrc/hp_attn.h, selects in place of the reference's
branches); tests/f16_round.hip compares it on the host with the oracle's
float32_to_float16 (lib.rs:2534-2569) for all 2^32 f32 bit patterns."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"


def test_f16_rounding_exhaustive(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None or not Path(HIPCC).exists():
        pytest.skip("gcc or hipcc not available")
    obj = tmp_path / "hp_oracle.o"
    subprocess.run([gcc, "-O2", "-c", str(ROOT / "oracle" / "hp_oracle.c"), "-o", str(obj)], check=True)
    main = tmp_path / "f16_round.o"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-c",
                    f"-I{ROOT / 'heliopause_amd' / 'csrc'}", str(ROOT / "tests" / "f16_round.hip"), "-o", str(main)],
                   check=True)
    exe = tmp_path / "f16_round"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-pthread", str(main), str(obj), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "f16 rounding mismatches 0" in r.stdout
