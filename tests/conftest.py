import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmunet_hip.so)")


def _gpu_count():
    import ctypes
    from munet_amd import _lib
    n = ctypes.c_int(0)
    try:
        _lib.call("mh_device_count", ctypes.byref(n))
    except Exception:
        return 0
    return n.value


@pytest.fixture(scope="session")
def hip():
    n = _gpu_count()
    if n == 0:
        pytest.skip("no GPU visible to the HIP runtime")
    import torch
    assert torch.cuda.is_available(), (
        f"HIP sees {n} device(s) but torch does not "
        f"(torch device count {torch._C._cuda_getDeviceCount()})")
    from munet_amd.backend import HipBackend
    return HipBackend(0)


@pytest.fixture(scope="session")
def orc():
    from oracle import CpuOracle, available
    if not available("restatement"):
        pytest.skip("oracle not built (make -C oracle)")
    return CpuOracle("restatement")
