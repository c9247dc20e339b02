"""GPU parity of the Q6 embedding path through the C ABI: the dequantizing
row gather (bit-exact: one rounding of fma(s, q, b)) and the decode token
tail with the next step's embedding row (bit-exact) and its RMSNorm (within
one bf16 ulp of the oracle's, whose sum of squares runs in another order)."""
import numpy as np
import pytest

from molten_amd import hip, layout
from tests.devutil import dev_quant, empty_dev, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("k", [2048, 1024])
def test_gather_rows_q6_bit_exact(dev, orc, k):
    _log(f"gather_rows_q6 k={k}")
    rng = np.random.default_rng(k)
    n, m = 4096, 37
    h = layout.synth_quant(rng, n, k, 6)
    ids = rng.integers(0, n, m).astype(np.uint32)
    ids[:3] = [0, n - 1, 0]
    dw, _keep = dev_quant(h)
    out = empty_dev((m, k), np.uint16)
    hip.gather_rows_q6(dw, to_dev(ids), m, out)
    np.testing.assert_array_equal(from_dev(out, np.uint16), orc.dequant_bf16(h)[ids])


def _ulps(a, b):
    ia = a.astype(np.int32)
    ib = b.astype(np.int32)
    oa = np.where(ia & 0x8000, 0x8000 - (ia & 0x7fff), 0x8000 + ia)
    ob = np.where(ib & 0x8000, 0x8000 - (ib & 0x7fff), 0x8000 + ib)
    return np.abs(oa - ob)


@pytest.mark.parametrize("k", [2048, 512])
def test_token_tail_embed(dev, orc, k):
    _log(f"token_tail_embed k={k}")
    rng = np.random.default_rng(k + 1)
    n, eps = 65536, 1e-5
    h = layout.synth_quant(rng, n, k, 6)
    w = layout.synth_bf16(rng, (k,), std=0.3)
    dw, _keep = dev_quant(h)
    for tok in (0, 12345, n - 1):
        key = (0x8000_1234 << 32) | (~tok & 0xffffffff)
        want_tok, want_x, want_n, _ = orc.token_tail_embed(key, h, w, eps)
        best = to_dev(np.array([key], np.uint64))
        out_tok = empty_dev((1,), np.uint32)
        x = empty_dev((k,), np.uint16)
        normed = empty_dev((k,), np.uint16)
        hip.token_tail_embed(best, out_tok, dw, to_dev(w), x, normed, eps)
        assert from_dev(out_tok, np.uint32)[0] == want_tok == tok
        assert from_dev(best, np.uint64)[0] == 0
        np.testing.assert_array_equal(from_dev(x, np.uint16), want_x)
        got = from_dev(normed, np.uint16)
        assert _ulps(got, want_n).max() <= 1
        g = layout.bf16_to_f32(got).astype(np.float64)
        r = layout.bf16_to_f32(want_n).astype(np.float64)
        assert np.linalg.norm(g - r) / np.linalg.norm(r) <= 5e-3


def test_token_tail_embed_empty_key(dev, orc):
    """An empty key (no argmax yet) gives token 0xffffffff and writes no rows."""
    rng = np.random.default_rng(5)
    h = layout.synth_quant(rng, 64, 2048, 6)
    dw, _keep = dev_quant(h)
    best = to_dev(np.zeros(1, np.uint64))
    out_tok = empty_dev((1,), np.uint32)
    x = to_dev(np.full(2048, 0x1234, np.uint16))
    normed = to_dev(np.full(2048, 0x1234, np.uint16))
    hip.token_tail_embed(best, out_tok, dw, to_dev(np.ones(2048, np.uint16)), x, normed, 1e-5)
    assert from_dev(out_tok, np.uint32)[0] == 0xffffffff
    assert (from_dev(x, np.uint16) == 0x1234).all() and (from_dev(normed, np.uint16) == 0x1234).all()
