import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


def gpu_available():
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    """cuda:0 with the native library loaded. On a machine with a GPU, a
    missing library fails the test instead of skipping it."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from dan_amd import _native

    _native.load()  # raises if the library is missing: no silent fallback
    return torch.device("cuda:0")
