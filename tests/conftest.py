import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libdsa.so")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests fail (not skip) when it is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible HIP device")
    from deberta_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
