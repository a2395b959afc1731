import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """Skips when no GPU is visible; fails loudly when a GPU is present but the
    HIP library was not built (there is no CPU fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from brush_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing on a GPU host: build it first")
    _lib.lib()
    return torch.device("cuda:0")
