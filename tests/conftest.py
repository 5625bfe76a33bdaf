import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from __graft_entry__ import load_package  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def pkg():
    """The esmfold2-mlx_amd package (directory name has a hyphen, so it is loaded by path)."""
    return load_package()


@pytest.fixture(scope="session")
def gpu_lib(pkg):
    """The loaded HIP library; fails loudly (no fallback) when it or the GPU is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    return pkg.capi.lib()
