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


# ---------------------------------------------------------------- kept set --

def _fkey(v):
    """Orderable u32 key of float32 values (-0 folded to +0)."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    u = np.where((u << np.uint64(1)) & np.uint64(0xffffffff) == 0, np.uint64(0), u)
    neg = (u & np.uint64(0x80000000)) != 0
    return np.where(neg, (~u) & np.uint64(0xffffffff), u | np.uint64(0x80000000)).astype(np.uint64)


def test_mass_target_is_exact_ceiling(orc):
    """The least integer >= top_p * z with top_p's exact f32 value."""
    from fractions import Fraction

    rng = np.random.default_rng(11)
    zs = [0, 1, 2, 3, 1 << 40, (1 << 57) - 1, 128000 << 40] + [int(z) for z in rng.integers(0, 1 << 57, 300)]
    ps = [0.5, 0.9, 0.95, 1e-3, 1e-30, 2.0 ** -126, 0.99999994] + list(rng.uniform(0, 1, 50))
    for p in ps:
        pf = Fraction(float(np.float32(p)))
        for z in zs:
            want = -((-pf * z).__floor__())  # ceiling
            assert orc.mass_target(z, float(np.float32(p))) == want, (p, z)


def test_mass_fixed_matches_float64(orc):
    rng = np.random.default_rng(12)
    m = 3.0
    for w in list(rng.uniform(-40, 3, 2000)) + [3.0, -100.0, -87.0]:
        w = float(np.float32(w))
        got = orc.mass_fixed(w, m)
        want = math.exp(float(np.float32(w - m))) * 2.0 ** 40
        assert got <= want * (1 + 3e-7) + 1 and got >= want * (1 - 3e-7) - 1, (w, got, want)
    assert orc.mass_fixed(m, m) == 1 << 40  # exp(0) = 1 exactly


def _w(logits, temp):
    return layout.bf16_to_f32(logits).astype(np.float32) * np.float32(1.0 / temp)


@pytest.mark.parametrize("k", [1, 2, 17, 500, 4095])
def test_topk_threshold_is_kth_largest(orc, k):
    """tau = the k-th largest w (numpy partition); ties at the boundary are
    kept (planted: the k-th value repeated around it)."""
    rng = np.random.default_rng(k)
    v = rng.normal(0, 2, 4096).astype(np.float32)
    order = np.argsort(-v)
    if k > 3:
        v[order[k - 3:k + 3]] = v[order[k - 1]]  # a tie group straddling k
    logits = layout.f32_to_bf16(v)
    w = _w(logits, 0.7)
    _, tau = orc.sample_draw(logits, None, float(np.float32(1 / 0.7)), 1.0, False, k, 1.0, 5, 0)
    kth = np.partition(w, len(w) - k)[len(w) - k]
    assert tau == int(_fkey(kth))
    kept = int((_fkey(w) >= tau).sum())
    assert kept >= k and kept == int((w >= kth).sum())


def test_topp_threshold_matches_float64(orc):
    """tau_p = the largest value t with softmax mass(w >= t) >= top_p, on
    logits whose cumulative masses are far from the boundary (float64)."""
    rng = np.random.default_rng(21)
    for trial in range(20):
        v = rng.normal(0, 3, 1000).astype(np.float32)
        logits = layout.f32_to_bf16(v)
        w = _w(logits, 1.0).astype(np.float64)
        vals = np.unique(w)[::-1]
        p = np.exp(w - w.max())
        p /= p.sum()
        cum = np.array([p[w >= t].sum() for t in vals])
        top_p = float(rng.uniform(0.3, 0.95))
        j = int(np.argmax(cum >= top_p))
        if abs(cum[j] - top_p) < 1e-4 or (j > 0 and abs(cum[j - 1] - top_p) < 1e-4):
            continue  # too close to call in float64 vs fixed point
        _, tau = orc.sample_draw(logits, None, 1.0, 1.0, False, 0, float(np.float32(top_p)), 1, trial)
        assert tau == int(_fkey(np.float32(vals[j]))), (trial, top_p)


def test_topk_then_topp(orc):
    """Both: top-p over the top-k set's own mass; tau >= tau_k."""
    rng = np.random.default_rng(31)
    v = rng.normal(0, 2, 2048).astype(np.float32)
    logits = layout.f32_to_bf16(v)
    w = _w(logits, 1.0).astype(np.float64)
    k, top_p = 50, 0.6
    kth = np.sort(w)[::-1][k - 1]
    sub = w[w >= kth]
    vals = np.unique(sub)[::-1]
    p = np.exp(sub - w.max())
    p /= p.sum()
    cum = np.array([p[sub >= t].sum() for t in vals])
    j = int(np.argmax(cum >= top_p))
    _, tau = orc.sample_draw(logits, None, 1.0, 1.0, False, k, top_p, 1, 0)
    assert tau == int(_fkey(np.float32(vals[j])))


def test_kept_set_reductions(orc):
    rng = np.random.default_rng(41)
    logits = layout.f32_to_bf16(rng.normal(0, 2, 4096).astype(np.float32))
    v = layout.bf16_to_f32(logits)
    greedy = int(np.argmax(v))
    for pos in range(8):
        # k = 1 and a tiny top_p keep only the max: the draw is greedy
        assert _token(orc.sample_draw(logits, None, 1.0, 1.0, False, 1, 1.0, 9, pos)[0]) == greedy
        assert _token(orc.sample_draw(logits, None, 1.0, 1.0, False, 0, 1e-6, 9, pos)[0]) == greedy
        # no top-k (k >= n is mapped to 0 by the host) and top_p = 1: the temperature draw
        assert (orc.sample_draw(logits, None, 1.25, 1.0, False, 0, 1.0, 9, pos)[0]
                == orc.sample_gumbel(logits, None, 1.25, 1.0, False, 9, pos))
        # top-k over every token keeps every token: the same draw
        assert (orc.sample_draw(logits, None, 1.25, 1.0, False, 4096, 1.0, 9, pos)[0]
                == orc.sample_gumbel(logits, None, 1.25, 1.0, False, 9, pos))


def test_kept_draw_follows_renormalized_softmax(orc):
    """Over many positions the draws are distributed as softmax(w)
    renormalized over the kept set, and never leave it."""
    logits = layout.f32_to_bf16(np.float32([0.0, 1.0, 2.0, -1.0, 0.5, 1.5, -2.0, 0.25]))
    w = layout.bf16_to_f32(logits).astype(np.float64)
    kept = np.argsort(-w)[:4]  # top_k = 4
    p = np.zeros(8)
    p[kept] = np.exp(w[kept] - w.max())
    p /= p.sum()
    n = 20000
    counts = np.zeros(8)
    for pos in range(n):
        counts[_token(orc.sample_draw(logits, None, 1.0, 1.0, False, 4, 1.0, 13, pos)[0])] += 1
    assert counts[p == 0].sum() == 0
    chi2 = float(((counts[kept] - n * p[kept]) ** 2 / (n * p[kept])).sum())
    assert chi2 < 25.0, (chi2, counts / n, p)  # df 3


def test_mass_of_infinite_and_nan_logits(orc):
    """w - m is NaN when both are the same infinity: the token then has the
    maximum's mass exp(0) = 2^40; a NaN w or m has none (so the top-p masses
    stay in [0, 2^40] for every input)."""
    inf = float("inf")
    assert orc.mass_fixed(-inf, -inf) == 1 << 40
    assert orc.mass_fixed(inf, inf) == 1 << 40
    assert orc.mass_fixed(-inf, 0.0) == 0
    assert orc.mass_fixed(1.0, inf) == 0
    assert orc.mass_fixed(float("nan"), 0.0) == 0
    assert orc.mass_fixed(0.0, float("nan")) == 0
    assert orc.mass_fixed(0.0, 0.0) == 1 << 40


@pytest.mark.parametrize("top_k,top_p", [(0, 0.9), (40, 0.5), (0, 1e-6)])
def test_all_minus_inf_logits_draw_like_the_temperature_draw(orc, top_k, top_p):
    """Every logit -inf: every token has the same key and mass, so top-k and
    top-p keep them all and the kept-set draw is the temperature draw (token
    0: every w + G is -inf and ties go to the lower id)."""
    n = 4096
    logits = np.full(n, 0xFF80, np.uint16)  # bf16 -inf
    for pos in range(3):
        key, tau = orc.sample_draw(logits, None, 1.0, 1.0, False, top_k, top_p, 5, pos)
        assert key == orc.sample_gumbel(logits, None, 1.0, 1.0, False, 5, pos)
        assert _token(key) == 0
        assert tau == int(_fkey(np.float32(-np.inf)))
