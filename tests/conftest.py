import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libgdn.so")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device for parity tests; fails (never skips) without one."""

    import torch

    assert torch.cuda.is_available(), "gpu-marked test run without a ROCm GPU"
    from mlx_lean_moe_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
