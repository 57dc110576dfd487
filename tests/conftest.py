import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the HIP library loaded; fails (does not skip) if the library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from laprune_amd import _native
    _native.lib()  # raises if the library is not built
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def orc():
    from oracle import orc as o
    o.lib()
    return o
