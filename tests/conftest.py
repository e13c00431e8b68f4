import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmiori_hip.so)")


@pytest.fixture(scope="session")
def dev():
    """The GPU; the HIP library must be built and loadable (no fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no GPU is visible")
    from miori_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
