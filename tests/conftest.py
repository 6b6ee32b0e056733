import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtrida_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device for parity tests. No skip: a GPU test run without a GPU is a failure."""
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a visible GPU (run with -m 'not gpu' on CPU-only hosts)")
    from trida_stack_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
