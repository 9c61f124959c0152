"""Test configuration: the ``gpu`` marker and shared fixtures.

Tests marked ``gpu`` need an MI355X (gfx950) and the built libhp_hip.so; they
compare the HIP path against the oracle (CPU restatement of the reference).
Everything else runs on the CPU.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def hip():
    """The HIP runner module; fails (never skips) when no GPU is usable."""
    from heliopause_amd import hip_kernels as H

    support = H.checkHipSupport()
    if not support["available"]:
        pytest.fail(f"HIP runner unavailable on a gpu-marked test: {support}")
    return H
