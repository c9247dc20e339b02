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


# Words every CU's LDS holds when a GPU test starts, rotated over the tests:
# LDS keeps what the previous kernel left, so a kernel that reads a word
# before writing it computes from these (large negative, NaN, all ones, large
# positive) and its outputs leave the oracle's.
_LDS_PATTERNS = (0xC7800000, 0x7FC00000, 0xFFFFFFFF, 0x47800000)
_lds_calls = [0]


@pytest.fixture(autouse=True)
def lds_garbage(request):
    """Before each GPU test: fill the LDS of every CU with a hostile word
    (libmolten_ceiling.so's mhc_lds_fill)."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    import ctypes

    import torch

    if not torch.cuda.is_available():
        yield
        return
    lib = ctypes.CDLL(os.path.join(ROOT, "molten_amd", "libmolten_ceiling.so"))
    lib.mhc_lds_fill.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    shift = int(os.environ.get("MH_TEST_LDS_SHIFT", "0"))  # another pattern per test in a second run
    pattern = _LDS_PATTERNS[(_lds_calls[0] + shift) % len(_LDS_PATTERNS)]
    _lds_calls[0] += 1
    assert lib.mhc_lds_fill(pattern, 4 * 256, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    yield
