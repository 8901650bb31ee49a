import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The torch device for GPU tests; the HIP library must be loadable."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from cast_amd import _lib
    _lib.load()          # raises if the library is missing: no silent fallback
    return torch.device("cuda:0")
