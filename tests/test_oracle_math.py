"""Pins the oracle's scalar pieces: bf16 conversion, exp, unpack/pack, the
argmax key and the exact FMA used by the replays."""
import math

import numpy as np
import pytest
import torch

from molten_amd import layout
from tests import exact


def test_bf16_to_f32_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = (h.astype(np.uint32) << 16).view(np.float32)
    got = np.array([orc.bf16_to_f32(int(v)) for v in h], dtype=np.float32)
    # ctypes returns a Python float (f64), which quiets signaling NaNs: compare
    # NaN patterns by NaN-ness, everything else bit for bit
    nan = np.isnan(ref)
    assert np.isnan(got[nan]).all()
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_bf16_matches_torch_rne(orc, rng):
    x = np.concatenate([
        rng.normal(0, 1, 20000).astype(np.float32),
        rng.normal(0, 1e30, 2000).astype(np.float32),
        rng.normal(0, 1e-38, 2000).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45], np.float32),
    ])
    # exact ties: low 16 bits == 0x8000, both parities of bit 16
    ties = (rng.integers(0, 2**15, 4000).astype(np.uint32) << 17 | 0x8000).view(np.float32)
    ties2 = ((rng.integers(0, 2**15, 4000).astype(np.uint32) << 17) | 0x18000).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)], ties2[np.isfinite(ties2)]])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got_np = layout.f32_to_bf16(x)
    np.testing.assert_array_equal(got_np, want)
    got_c = np.array([orc.f32_to_bf16(float(v)) for v in x[::3]], np.uint16)
    np.testing.assert_array_equal(got_c, want[::3])


def test_f32_to_bf16_nan_is_quiet(orc):
    for bits in (0x7F800001, 0xFF800001, 0x7FC00000, 0x7F80FFFF):
        v = np.array([bits], np.uint32).view(np.float32)[0]
        r = orc.f32_to_bf16(float(v))
        assert (r & 0x7F80) == 0x7F80 and (r & 0x7F) != 0


def _ulp_err(got: np.ndarray, ref: np.ndarray) -> np.ndarray:
    sp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref) / sp


def test_expf_accuracy(orc):
    x = np.concatenate([
        np.linspace(-87.0, 88.7, 60001, dtype=np.float32),
        np.linspace(-2, 2, 20001, dtype=np.float32),
    ])
    got = orc.expf_array(x)
    ref = np.exp(x.astype(np.float64))
    assert _ulp_err(got, ref).max() <= 2.0


def test_expf_special_values(orc):
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-0.0) == 1.0
    assert orc.expf(float("inf")) == float("inf")
    assert orc.expf(float("-inf")) == 0.0
    assert math.isnan(orc.expf(float("nan")))
    assert orc.expf(89.0) == float("inf")
    assert orc.expf(-110.0) == 0.0
    # denormal results: within one denormal step of the true value
    for v in (-88.0, -95.0, -100.0, -103.0):
        assert abs(orc.expf(v) - math.exp(v)) <= 2 ** -149


def test_sigmoid_score_drops_at_most_half_ulp(orc):
    """The sigmoid routing score 1 / (1 + expf(-z)) over every float z in
    increasing order never falls more than 2^-24 below its running maximum
    (exhaustive, 4.3e9 values; the defect comes from the exp's reduction
    boundaries).  The matrix-core prefill router widens its score bounds by
    this amount; the test also checks the drop is not zero, i.e. that the
    scan does see the function's defect."""
    d = orc.sigmoid_max_drop()
    assert 0.0 < d <= 2.0 ** -24, d


def test_unpack_known_answers(orc):
    np.testing.assert_array_equal(orc.unpack(np.array([0x76543210], np.uint32), 4, 8),
                                  np.arange(8))
    # Q6 packet [1, 2, 3, 4] -> bytes 0x81 0x30 0x10 (lfm.metal:186-199)
    packed = orc.pack(np.array([1, 2, 3, 4] * 4, np.uint8), 6)
    assert packed.view(np.uint8)[:3].tolist() == [0x81, 0x30, 0x10]
    np.testing.assert_array_equal(orc.unpack(packed, 6, 16), [1, 2, 3, 4] * 4)


@pytest.mark.parametrize("bits", [4, 6, 8])
def test_pack_unpack_roundtrip_and_numpy_agree(orc, rng, bits):
    k = 256
    q = rng.integers(0, 2**bits, size=(5, k), dtype=np.uint8)
    codes_np = layout.pack_codes(q, bits)
    for r in range(5):
        np.testing.assert_array_equal(orc.pack(q[r], bits), codes_np[r])
        np.testing.assert_array_equal(orc.unpack(codes_np[r], bits, k), q[r])
    np.testing.assert_array_equal(layout.unpack_codes(codes_np, bits, k), q)


def test_q6_matches_reference_byte_formula(rng):
    # lfm.metal:186-199: q0=b0&63, q1=(b0>>6)|((b1&15)<<2), q2=(b1>>4)|((b2&3)<<4), q3=b2>>2
    q = rng.integers(0, 64, size=(1, 64), dtype=np.uint8)
    b = layout.pack_codes(q, 6).view(np.uint8).reshape(-1, 3).astype(int)
    dec = np.stack([b[:, 0] & 63, (b[:, 0] >> 6) | ((b[:, 1] & 15) << 2),
                    (b[:, 1] >> 4) | ((b[:, 2] & 3) << 4), b[:, 2] >> 2], axis=1).ravel()
    np.testing.assert_array_equal(dec, q[0])


def test_argmax_key_orders_like_merge(orc, rng):
    vals = np.concatenate([rng.normal(0, 10, 300), [0.0, -0.0, np.inf, -np.inf, 1.0, 1.0]])
    vals = vals.astype(np.float32)
    idx = rng.integers(0, 1000, vals.size)
    for _ in range(3000):
        i, j = rng.integers(0, vals.size, 2)
        vi, vj, ii, ij = vals[i], vals[j], int(idx[i]), int(idx[j])
        ki, kj = orc.argmax_key(float(vi), ii), orc.argmax_key(float(vj), ij)
        i_wins = vi > vj or (vi == vj and ii < ij)
        j_wins = vj > vi or (vi == vj and ij < ii)
        if i_wins:
            assert ki > kj
        elif j_wins:
            assert kj > ki
        else:
            assert ki == kj


def test_argmax_known_answers(orc):
    f = layout.f32_to_bf16
    assert orc.argmax_bf16(f(np.array([1, 3, 3, 2], np.float32))) == 1
    assert orc.argmax_bf16(f(np.array([-0.0, 0.0, -1.0], np.float32))) == 0
    assert orc.argmax_bf16(f(np.array([-1.0, -0.0, 0.0], np.float32))) == 1
    assert orc.argmax_bf16(f(np.full(5, -np.inf, np.float32))) == 0
    assert orc.argmax_bf16(f(np.array([np.nan, 1.0, np.nan, 2.0], np.float32))) == 3
    assert orc.argmax_bf16(f(np.array([np.nan, np.nan], np.float32))) == 0


def test_exact_fma_against_float64_when_exact(rng):
    # when a*b + c is exactly representable in f64, f64 then f32 rounding is a
    # single rounding: the exact FMA must agree
    for _ in range(2000):
        a, b = np.float32(rng.integers(-4096, 4096)), np.float32(rng.normal())
        c = np.float32(rng.normal())
        assert exact.fma32(a, b, c) == np.float32(np.float64(a) * np.float64(b) + np.float64(c))
    # a classic double-rounding case where fma differs from mul-then-add
    a = np.float32(1.0 + 2.0 ** -12)
    got = exact.fma32(a, a, np.float32(-1.0))
    assert got == np.float32(2.0 ** -11 + 2.0 ** -24)
    assert exact.mul32(a, a) - np.float32(1.0) != got
