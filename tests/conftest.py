import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "deepseek-v41-mlx_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    """GPU tests fail loudly (not skip) when no GPU is present but were explicitly selected;
    unselected runs (-m "not gpu") never reach them."""
    return


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but torch sees no GPU")
    from dsv41 import _abi
    _abi.lib()  # raises if libdsv41.so is missing: no silent fallback
    return torch.device("cuda:0")
