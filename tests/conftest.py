"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X (or any HIP device) and the built
libraries; everything else runs on the CPU.  The repository root is put on
sys.path so ``rushlite_amd`` and ``oracle`` import without installation.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU and the built backend")


def gpu_available() -> bool:
    try:
        from rushlite_amd import abi
        import ctypes
        n = ctypes.c_int(0)
        abi.lib().lmp_rt_device_count(ctypes.byref(n))
        return n.value > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip():
    """The C-ABI binding, initialised on device 0 (GPU tests only)."""
    from rushlite_amd import abi
    if not gpu_available():
        pytest.fail("no HIP device visible to a test marked gpu")
    abi.check(abi.lib().lmp_rt_init(0))
    return abi


@pytest.fixture(scope="session")
def oracle():
    from oracle import lamp_oracle
    lamp_oracle.load()
    return lamp_oracle
