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


def _keys_f32(v):
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    u = np.where((u << np.uint64(1)) & np.uint64(0xffffffff) == 0, np.uint64(0), u)
    neg = (u & np.uint64(0x80000000)) != 0
    return np.where(neg, (~u) & np.uint64(0xffffffff), u | np.uint64(0x80000000))


@pytest.mark.parametrize("n,temp,penalty,top_k,top_p,seed,pos", [
    (128000, 1.0, 1.0, 40, 1.0, 7, 0),         # top-k only
    (128000, 0.8, 1.0, 0, 0.9, 11, 3),         # top-p only
    (128000, 0.7, 1.3, 50, 0.95, 2 ** 40 + 3, 99),  # both, with the repetition penalty
    (128000, 1.2, 1.0, 1, 1.0, 5, 12),         # k = 1: greedy
    (128000, 1.0, 1.0, 0, 1e-6, 5, 13),        # tiny top_p: greedy
    (128000, 1.0, 1.0, 127999, 1.0, 5, 14),    # k = n - 1
    (4096, 2.0, 1.0, 300, 0.5, 123, 77),       # a partial last workgroup? (4096 = 4 whole ones)
    (1000, 0.9, 1.0, 10, 0.8, 9, 5),           # a partial workgroup
])
def test_sample_draw_bit_exact(dev, orc, n, temp, penalty, top_k, top_p, seed, pos):
    """The kept-set draw's key equals the oracle's bit for bit (integer
    thresholds: counts and fixed-point masses; the draw as the temperature
    draw), over repeated calls on one workspace whose scratch part starts as
    garbage and whose head (hip.SAMPLE_ZERO_BYTES) is left zero."""
    rng = np.random.default_rng(n + top_k + pos)
    v = rng.normal(0, 3, n).astype(np.float32)
    # ties around the k-th largest and exact zeros
    order = np.argsort(-v)
    if 3 < top_k < n - 3:
        v[order[top_k - 3:top_k + 3]] = v[order[top_k - 1]]
    v[:4] = [0.0, -0.0, 0.0, 1e-3]
    logits = layout.f32_to_bf16(v)
    seen = rng.integers(0, 2 ** 32, (n + 31) // 32, dtype=np.uint64).astype(np.uint32)
    use_pen = penalty != 1.0
    ws_bytes = hip.sample_workspace_bytes(n)
    # only the head must start at zero: the rest holds garbage
    ws_host = np.full(ws_bytes, 0xA5, np.uint8)
    ws_host[:hip.SAMPLE_ZERO_BYTES] = 0
    ws = to_dev(ws_host)
    dl, ds = to_dev(logits), to_dev(seen)
    for call in range(3):
        p = hip.sample_params(temp, seed, pos + call, penalty, top_k, top_p)
        want, tau = orc.sample_draw(logits, seen if use_pen else None, p.inv_temp, penalty, use_pen, top_k,
                                    p.top_p, seed, pos + call)
        best = to_dev(np.zeros(1, np.uint64))
        hip.sample_draw(dl, n, ds, p, best, ws, ws_bytes)
        got = int(from_dev(best, np.uint64)[0])
        assert got == want, (call, hex(got), hex(want))
        assert not from_dev(ws, np.uint8)[:hip.SAMPLE_ZERO_BYTES].any()  # counters and round 0's bins left zero
    # the drawn token is in the kept set
    w = layout.bf16_to_f32(logits).astype(np.float32) * np.float32(p.inv_temp)
    tok = (~got) & 0xffffffff
    assert use_pen or _keys_f32(w[tok]) >= tau


@pytest.mark.parametrize("n,top_k,top_p,levels,seed", [
    (128000, 1000, 0.9, 0, 21),   # a kept list longer than the finishing workgroup takes
    (128000, 40, 0.5, 24, 22),    # few distinct values: thousands tied at the k-th largest
    (128000, 200, 0.99, 0, 23),   # a list below the cap
    (4096, 4095, 0.7, 8, 24),     # nearly every token kept, ties
])
def test_sample_draw_kept_list_and_ties(dev, orc, n, top_k, top_p, levels, seed):
    """top-k with top-p: the mass phase decided over the kept list by the
    draw's last workgroup, and, when the list is longer than it takes (large
    k, or ties at the threshold), by its own radix rounds over every token;
    bit for bit against the oracle over two calls on one workspace."""
    rng = np.random.default_rng(seed)
    v = rng.normal(0, 3, n).astype(np.float32)
    if levels:
        v = np.round(v * levels / 8.0) * np.float32(8.0 / levels)
    logits = layout.f32_to_bf16(v.astype(np.float32))
    seen = np.zeros((n + 31) // 32, np.uint32)
    ws_bytes = hip.sample_workspace_bytes(n)
    ws_host = np.full(ws_bytes, 0x5A, np.uint8)
    ws_host[:hip.SAMPLE_ZERO_BYTES] = 0
    ws = to_dev(ws_host)
    dl, ds = to_dev(logits), to_dev(seen)
    for call in range(2):
        p = hip.sample_params(1.0, seed, call, 1.0, top_k, top_p)
        want, tau = orc.sample_draw(logits, None, p.inv_temp, 1.0, False, top_k, p.top_p, seed, call)
        best = to_dev(np.zeros(1, np.uint64))
        hip.sample_draw(dl, n, ds, p, best, ws, ws_bytes)
        got = int(from_dev(best, np.uint64)[0])
        assert got == want, (call, hex(got), hex(want))
        assert not from_dev(ws, np.uint8)[:hip.SAMPLE_ZERO_BYTES].any()


def test_sample_mark_sets_the_bit(dev):
    seen = to_dev(np.zeros(4000, np.uint32))
    for t in (0, 31, 32, 127999, 128000, 5000000):
        hip.sample_mark(to_dev(np.uint32([t])), seen, 128000)
    got = from_dev(seen, np.uint32)
    want = np.zeros(4000, np.uint32)
    for t in (0, 31, 32, 127999):
        want[t >> 5] |= np.uint32(1 << (t & 31))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n,top_k,top_p", [(128000, 0, 0.9), (128000, 40, 0.5), (4096, 0, 1e-6)])
def test_sample_draw_all_minus_inf(dev, orc, n, top_k, top_p):
    """Every logit -inf with top-k / top-p on: the masses are defined (every
    token the maximum's), the kept set is every token and the draw's key is
    the oracle's, which is the temperature draw's (token 0)."""
    logits = np.full(n, 0xFF80, np.uint16)
    seen = np.zeros((n + 31) // 32, np.uint32)
    ws_bytes = hip.sample_workspace_bytes(n)
    ws = to_dev(np.zeros(ws_bytes, np.uint8))
    dl, ds = to_dev(logits), to_dev(seen)
    for call in range(2):
        p = hip.sample_params(1.0, 17, call, 1.0, top_k, top_p)
        want, _ = orc.sample_draw(logits, None, p.inv_temp, 1.0, False, top_k, p.top_p, 17, call)
        assert want == orc.sample_gumbel(logits, None, p.inv_temp, 1.0, False, 17, call)
        best = to_dev(np.zeros(1, np.uint64))
        hip.sample_draw(dl, n, ds, p, best, ws, ws_bytes)
        got = int(from_dev(best, np.uint64)[0])
        assert got == want, (call, hex(got), hex(want))
        assert (~got) & 0xFFFFFFFF == 0
        assert not from_dev(ws, np.uint8)[:hip.SAMPLE_ZERO_BYTES].any()
