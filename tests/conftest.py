import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(GOLDEN / name, allow_pickle=False)
    return load


@pytest.fixture(scope="session")
def codebooks(golden):
    return golden("codebooks.npz")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests fail (not skip) when it or the library is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible HIP device"
    from sub0_amd import _native
    _native.lib()
    return torch.device("cuda:0")
