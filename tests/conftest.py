import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the GPU)")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """The GPU test device.  Skips only when no GPU is visible; a missing or
    broken native library is a failure, never a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from molten_amd import hip

    hip.load()
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
