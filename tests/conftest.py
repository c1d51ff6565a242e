import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvortx_hip.so on the device)")


def _require_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU (run with -m 'not gpu')")


@pytest.fixture(scope="session")
def gemm():
    _require_gpu()
    import vortx_amd as vx
    return vx.Gemm(0)


@pytest.fixture(scope="session")
def qgemv():
    _require_gpu()
    import vortx_amd as vx
    return vx.QuantGemv(0)
