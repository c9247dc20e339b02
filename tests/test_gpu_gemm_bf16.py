"""The dense bf16 GEMM (src/kernels/gemm.rs:33 gemm_bf16_nt), the generic
quantized GEMM (src/kernels/quant.rs:126 gemm_quant_bf16_nt) and the 8-bit
dequantization (quant.rs:69 with bits 8) through the C ABI.

C = A . B^T is checked against float64 numpy on the same bf16 operands (the
stated tolerance, literal errors printed) and exactly on one-hot rows of A
(C[m, n] = B[n, k_m], a bf16 value: every product but one is zero, so any
accumulation order gives it).  The dequantization is bit-exact against the
oracle."""
import numpy as np
import pytest

from molten_amd import hip, layout
from tests.devutil import assert_tolerance, dev_quant, empty_dev, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _gemm_ref(a, b):
    af = layout.bf16_to_f32(a).astype(np.float64)
    bf = layout.bf16_to_f32(b).astype(np.float64)
    return af @ bf.T


@pytest.mark.parametrize("m,n,k", [
    (4096, 2048, 2048),   # a prefill attention projection (256-row tiles)
    (2085, 4160, 192),    # ragged M and N on the 256-row tiles (297 tiles)
    (300, 200, 1536),     # ragged M and N on the 128-row tiles
    (128, 128, 64),       # one tile, one k block
    (33, 17, 40),         # K % 64 != 0: the per-element path
    (5, 11776, 192),      # few rows, wide N
])
def test_gemm_bf16_nt_matches_float64(dev, m, n, k):
    print(f"gemm_bf16_nt m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = layout.synth_bf16(rng, (m, k))
    b = layout.synth_bf16(rng, (n, k), std=0.05)
    c = empty_dev((m, n), np.uint16)
    hip.gemm_bf16_nt(to_dev(a), to_dev(b), c, m, n, k)
    assert_tolerance(from_dev(c, np.uint16), _gemm_ref(a, b), f"gemm_bf16_nt {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(256, 384, 2048), (2085, 4160, 128), (70, 50, 128), (9, 13, 72)])
def test_gemm_bf16_nt_one_hot_exact(dev, m, n, k):
    """One-hot rows of A pick columns of B exactly (any summation order)."""
    rng = np.random.default_rng(k + m)
    b = layout.synth_bf16(rng, (n, k))
    pick = rng.integers(0, k, m)
    a = np.zeros((m, k), np.uint16)
    a[np.arange(m), pick] = layout.f32_to_bf16(np.ones(1, np.float32))[0]
    c = empty_dev((m, n), np.uint16)
    hip.gemm_bf16_nt(to_dev(a), to_dev(b), c, m, n, k)
    got = from_dev(c, np.uint16)
    want = b[:, pick].T
    # a -0 entry of B gives -0 + (+0 products) = +0 in any order: compare values
    np.testing.assert_array_equal(np.where(want == 0x8000, 0, want), np.where(got == 0x8000, 0, got))


def test_gemm_bf16_nt_unaligned_operands(dev):
    """Operands offset by one element (not 16-byte aligned) take the
    per-element path and still match."""
    rng = np.random.default_rng(3)
    m, n, k = 40, 24, 128
    a = layout.synth_bf16(rng, (m * k + 1,))
    b = layout.synth_bf16(rng, (n * k + 1,))
    da, db = to_dev(a), to_dev(b)
    c = empty_dev((m, n), np.uint16)
    hip.gemm_bf16_nt(da.data_ptr() + 2, db.data_ptr() + 2, c, m, n, k)
    want = _gemm_ref(a[1:].reshape(m, k), b[1:].reshape(n, k))
    assert_tolerance(from_dev(c, np.uint16), want, "gemm_bf16_nt unaligned")


@pytest.mark.parametrize("bits", [4, 6, 8])
def test_dequant_bit_exact_all_widths(dev, orc, bits):
    rng = np.random.default_rng(40 + bits)
    h = layout.synth_quant(rng, 96, 1024, bits)
    w, keep = dev_quant(h)
    out = empty_dev((96, 1024), np.uint16)
    hip.dequant_to_bf16(w, out)
    np.testing.assert_array_equal(from_dev(out, np.uint16), orc.dequant_bf16(h))


@pytest.mark.parametrize("bits", [4, 6, 8])
@pytest.mark.parametrize("m", [1, 37, 512])
def test_gemm_quant_bf16_nt(dev, orc, bits, m):
    """dequantize into the scratch, then the GEMM: the scratch holds the
    oracle's dequantized W bit for bit, C is within tolerance of float64 over
    those values, and exact on one-hot rows."""
    print(f"gemm_quant_bf16_nt bits={bits} m={m}", flush=True)
    rng = np.random.default_rng(bits * 100 + m)
    n, k = 768, 2048
    h = layout.synth_quant(rng, n, k, bits)
    w, keep = dev_quant(h)
    wq = orc.dequant_bf16(h)
    a = layout.synth_bf16(rng, (m, k))
    rows = min(m, 2)
    pick = rng.integers(0, k, rows)
    a[:rows] = 0
    a[np.arange(rows), pick] = layout.f32_to_bf16(np.ones(1, np.float32))[0]
    scratch = empty_dev((n * k + 64,), np.uint16)
    c = empty_dev((m, n), np.uint16)
    hip.gemm_quant_bf16_nt(to_dev(a), m, w, c, scratch, n * k + 64)
    np.testing.assert_array_equal(from_dev(scratch, np.uint16)[:n * k].reshape(n, k), wq)
    got = from_dev(c, np.uint16)
    np.testing.assert_array_equal(got[:rows], wq[:, pick].T)
    assert_tolerance(got, _gemm_ref(a, wq), f"gemm_quant_bf16_nt bits={bits} m={m}")
