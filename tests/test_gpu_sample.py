"""GPU parity of the temperature-only Gumbel draw through the C ABI: the
folded key equals the oracle's bit for bit (Philox is integer, the log is the
library's own, every float step is IEEE in one order)."""
import numpy as np
import pytest

from molten_amd import hip, layout
from tests.devutil import from_dev, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("temp,penalty,seed,pos", [
    (1.0, 1.0, 0, 0), (0.7, 1.3, 12345678901, 77), (1.6, 1.0, 2 ** 63 + 5, 4095), (0.05, 2.0, 9, 1 << 20),
])
def test_sample_gumbel_bit_exact(dev, orc, temp, penalty, seed, pos):
    rng = np.random.default_rng(seed & 0xffff)
    n = 128000  # the reference's vocabulary
    logits = layout.f32_to_bf16(rng.normal(0, 3, n).astype(np.float32))
    logits[:8] = layout.f32_to_bf16(np.float32([0.0, -0.0, 5.0, 5.0, -1.0, 0.0, 1e-3, -1e-3]))
    seen = rng.integers(0, 2 ** 32, n // 32, dtype=np.uint64).astype(np.uint32)
    p = hip.sample_params(temp, seed, pos, penalty)
    want = orc.sample_gumbel(logits, seen if penalty != 1.0 else None, p.inv_temp, penalty, penalty != 1.0,
                             seed, pos)
    best = to_dev(np.zeros(1, np.uint64))
    hip.sample_gumbel(to_dev(logits), n, to_dev(seen), p, best)
    assert int(from_dev(best, np.uint64)[0]) == want
    # a second draw folds into the key word (max), as the reference's atomic max does
    p2 = hip.sample_params(temp, seed, pos + 1, penalty)
    want2 = orc.sample_gumbel(logits, seen if penalty != 1.0 else None, p.inv_temp, penalty, penalty != 1.0,
                              seed, pos + 1, best=want)
    hip.sample_gumbel(to_dev(logits), n, to_dev(seen), p2, best)
    assert int(from_dev(best, np.uint64)[0]) == want2
