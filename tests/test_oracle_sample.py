"""Pins the oracle's temperature-only Gumbel draw (lfm_sample.metal:124-190):
Philox4x32-10 against Random123's published known-answer vectors, the own
log against float64, the Gumbel transform against float64, and the draw's
distribution against softmax(w) (the Gumbel-max trick)."""
import math

import numpy as np
import pytest

from molten_amd import layout


@pytest.mark.parametrize("ctr,key,want", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(orc, ctr, key, want):
    assert orc.philox(ctr, key).tolist() == want


def _ulp(x):
    return np.spacing(np.float32(abs(x))).astype(np.float64)


def test_logf_within_two_ulp(orc):
    rng = np.random.default_rng(0)
    xs = np.concatenate([np.exp(rng.uniform(-87, 88, 20000)).astype(np.float32),
                         np.float32([1e-45, 1e-40, 1.17549435e-38, 0.5, 1.0, 2.0, 1.41421354, 1.41421366,
                                     3.4e38, 1 - 2 ** -24, 1 + 2 ** -23])])
    worst = 0.0
    for x in xs:
        got = orc.logf(float(x))
        want = math.log(float(x))
        worst = max(worst, abs(got - want) / float(_ulp(want) if want != 0 else 1e-45))
    assert worst <= 2.0, worst
    assert orc.logf(1.0) == 0.0
    for k in range(-126, 128, 7):  # exact powers of two: k ln2 within an ulp
        assert abs(orc.logf(2.0 ** k) - k * math.log(2.0)) <= float(_ulp(k * math.log(2.0))) * 1.0 + 1e-45


def test_gumbel_transform(orc):
    xs = [0, 1, 2 ** 20, 2 ** 26 - 1, 2 ** 26, 2 ** 26 + 1, 2 ** 31, 2 ** 32 - 2 ** 8, 2 ** 32 - 1]
    xs += list(np.random.default_rng(1).integers(0, 2 ** 32, 2000))
    for x in xs:
        # V as the f32 formula rounds it; then float64 from there on
        v = float(np.float32(np.float32(np.float32(x) + np.float32(0.5)) * np.float32(2.0 ** -32)))
        if v < 0.015625:
            want = -math.log(-math.log1p(-v))
        else:
            want = -math.log(-math.log(max(float(np.float32(1.0) - np.float32(v)), 2.0 ** -25)))
        got = orc.gumbel(int(x))
        assert abs(got - want) <= 1e-5 * max(1.0, abs(want)), (x, got, want)


def _token(key):
    return (~key) & 0xffffffff


def test_draw_follows_softmax(orc):
    """Over many positions the draws of one row are distributed as softmax(w)."""
    logits = layout.f32_to_bf16(np.float32([0.0, 1.0, 2.0, -1.0, 0.5, 1.5, -2.0, 0.25]))
    temp = 0.8
    w = layout.bf16_to_f32(logits).astype(np.float64) / temp
    p = np.exp(w - w.max())
    p /= p.sum()
    n = 40000
    counts = np.zeros(8)
    for pos in range(n):
        counts[_token(orc.sample_gumbel(logits, None, float(np.float32(1 / temp)), 1.0, False, 7, pos))] += 1
    chi2 = float(((counts - n * p) ** 2 / (n * p)).sum())
    assert chi2 < 30.0, (chi2, counts / n, p)  # df 7: p-value ~1e-4


def test_draw_closed_forms(orc):
    rng = np.random.default_rng(2)
    logits = layout.f32_to_bf16(rng.normal(0, 2, 4096).astype(np.float32))
    v = layout.bf16_to_f32(logits)
    greedy = int(np.argmax(v))
    # near-zero temperature: the noise cannot move the argmax
    for pos in range(5):
        assert _token(orc.sample_gumbel(logits, None, 1e4, 1.0, False, 3, pos)) == greedy
    # a huge repetition penalty on the greedy token (positive logit) drops it
    seen = np.zeros(4096 // 32, np.uint32)
    seen[greedy >> 5] |= np.uint32(1 << (greedy & 31))
    second = int(np.argsort(v)[-2])
    assert v[greedy] > 0
    for pos in range(5):
        assert _token(orc.sample_gumbel(logits, seen, 1e4, 1e30, True, 3, pos)) == second
    # folding: a key already above every draw is kept
    top = (0xffffffff << 32) | 0xfffffff0
    assert orc.sample_gumbel(logits, None, 1.0, 1.0, False, 3, 0, best=top) == top
