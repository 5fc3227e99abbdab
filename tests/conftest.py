import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmunet_hip.so)")


@pytest.fixture(scope="session")
def hip():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from munet_amd.backend import HipBackend
    return HipBackend(0)


@pytest.fixture(scope="session")
def orc():
    from oracle import CpuOracle, available
    if not available("restatement"):
        pytest.skip("oracle not built (make -C oracle)")
    return CpuOracle("restatement")
