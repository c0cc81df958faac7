import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """Skip-free GPU fixture: GPU tests are selected with -m gpu and must fail
    loudly, not skip, when the device or the HIP library is missing."""
    import torch
    assert torch.cuda.is_available(), "gpu-marked test needs a visible GPU"
    from fastalgebraictransformer_amd import _lib
    _lib.load()
    return torch.device("cuda:0")
