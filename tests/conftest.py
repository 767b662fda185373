import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libllamatov_hip.so")
    config.addinivalue_line("markers", "slow: long-running (full-size model) test")


def _gpu_available() -> bool:
    try:
        import ctypes
        from llamatov_amd import _lib
        lib = _lib.load()
        n = ctypes.c_int(0)
        return lib.lt_device_count(ctypes.byref(n)) == 0 and n.value > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The shared device context; fails (not skips) when the HIP library is missing, so a
    GPU run can never pass on a silent fallback."""
    from llamatov_amd import engine as dr
    if not _gpu_available():
        pytest.fail("no usable gfx950 device / libllamatov_hip.so for a gpu-marked test")
    return dr.get_device()


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as orc
    orc.lib()
    return orc
