import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libcgpt.so")


@pytest.fixture(scope="session")
def gpu():
    """Skip when no GPU is visible; fail loudly when the kernel library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from cutilegpt_amd import _lib
    _lib.load()  # raises KernelLibraryError: no silent fallback
    return torch.device("cuda:0")
