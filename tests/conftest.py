import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libdiagpu.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle import binding
    binding.lib()
    return binding


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with libdiagpu.so loaded; a missing library is a failure."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from diagpu_amd import _lib
    _lib.load()
    return torch.device("cuda:0")
