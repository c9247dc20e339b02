"""GPU parity of the decode GEMV epilogue variants through the C ABI:
proj3_gemv_scatter (Q, K, V projections, V into the KV cache) and
conv3_gemv (short-conv projection + conv).  The row values follow the
oracle's chunk order, so every output is bit-exact."""
import numpy as np
import pytest

from molten_amd import hip, layout
from tests.devutil import dev_quant, from_dev, to_dev, empty_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("k,nq,nk,nv,max_seq,pos", [
    (2048, 2048, 512, 512, 64, 5),   # the model's attention projections (8 KV heads of 64)
    (1024, 100, 24, 128, 3, 2),      # partial row blocks, K below 2048
])
def test_proj3_bit_exact(dev, orc, k, nq, nk, nv, max_seq, pos):
    _log(f"proj3 k={k} nq={nq} nk={nk} nv={nv}")
    rng = np.random.default_rng(nq + nk)
    hq, hk, hv = (layout.synth_quant(rng, n, k, 4) for n in (nq, nk, nv))
    x = layout.synth_bf16(rng, (1, k))[0]
    cache = layout.synth_bf16(rng, (nv // 64, max_seq, 64))
    want_cache = cache.copy()
    want_q, want_k = orc.proj3(hq, hk, hv, x, max_seq, pos, want_cache)
    (dq, _kq), (dk, _kk), (dv, _kv) = dev_quant(hq), dev_quant(hk), dev_quant(hv)
    q = empty_dev((nq,), np.uint16)
    kk = empty_dev((nk,), np.uint16)
    dc = to_dev(cache)
    hip.proj3_gemv_scatter(dq, dk, dv, to_dev(x), q, kk, dc, max_seq, pos)
    np.testing.assert_array_equal(from_dev(q, np.uint16), want_q)
    np.testing.assert_array_equal(from_dev(kk, np.uint16), want_k)
    np.testing.assert_array_equal(from_dev(dc, np.uint16), want_cache)


@pytest.mark.parametrize("H,k", [(2048, 2048), (100, 1024)])
def test_conv3_bit_exact(dev, orc, H, k):
    _log(f"conv3 H={H} k={k}")
    rng = np.random.default_rng(H)
    h = layout.synth_quant(rng, 3 * H, k, 4)
    x = layout.synth_bf16(rng, (1, k))[0]
    taps = layout.synth_bf16(rng, (H, 3), std=0.5)
    state = layout.synth_bf16(rng, (2, H))
    want_out, want_state = orc.conv3(h, x, taps, state)
    dw, _keep = dev_quant(h)
    out = empty_dev((H,), np.uint16)
    new_state = empty_dev((2, H), np.uint16)
    hip.conv3_gemv(dw, to_dev(x), to_dev(taps), to_dev(state), out, new_state)
    np.testing.assert_array_equal(from_dev(out, np.uint16), want_out)
    np.testing.assert_array_equal(from_dev(new_state, np.uint16), want_state)


def test_conv3_state_in_place(dev, orc):
    """new_state may be the state buffer itself (each channel reads before it writes)."""
    H, k = 256, 2048
    rng = np.random.default_rng(7)
    h = layout.synth_quant(rng, 3 * H, k, 4)
    x = layout.synth_bf16(rng, (1, k))[0]
    taps = layout.synth_bf16(rng, (H, 3), std=0.5)
    state = layout.synth_bf16(rng, (2, H))
    want_out, want_state = orc.conv3(h, x, taps, state)
    dw, _keep = dev_quant(h)
    out = empty_dev((H,), np.uint16)
    ds = to_dev(state)
    hip.conv3_gemv(dw, to_dev(x), to_dev(taps), ds, out, ds)
    np.testing.assert_array_equal(from_dev(out, np.uint16), want_out)
    np.testing.assert_array_equal(from_dev(ds, np.uint16), want_state)
