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
    """The GPU tests run the HIP library or fail: no skip, no fallback."""
    import torch

    import kyro_amd

    assert torch.cuda.is_available(), "gpu-marked test collected on a machine without a GPU"
    kyro_amd.lib()  # raises ImportError if libkyro_verify.so was not built
    return torch.device("cuda", 0)
