import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) GPU and the built library")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device, with libffai_attn.so loaded. A GPU test never falls back: a missing library
    is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from ffai_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
