import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs on the GPU box)")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library loaded next to torch on cuda:0; fails loudly (no
    fallback) when the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    from gpu_offloading_amd import _lib

    _lib.load()
    torch.cuda.set_device(0)
    return torch.device("cuda:0")
