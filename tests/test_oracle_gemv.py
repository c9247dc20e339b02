"""Pins the oracle's GEMV family (a4, a5, a6, a7) and dequant."""
import numpy as np
import pytest

from molten_amd import layout
from tests import exact

bf = layout.bf16_to_f32


def _ulps_bf16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 arrays (monotone integer map)."""
    def key(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, 0x8000 - (h & 0x7FFF), 0x8000 + h)
    return np.abs(key(a) - key(b))


@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("n,k,batch", [(64, 2048, 1), (40, 1536, 2), (16, 4096, 3)])
def test_gemv_matches_float64(orc, rng, bits, n, k, batch):
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    y, yf = orc.gemv_quant(h, x, batch, want_f32=True)
    ref = bf(x).astype(np.float64) @ h.dequant_f64().T
    # f32 accumulation of ~k terms: relative error well below one bf16 ulp
    scale = np.abs(bf(x).astype(np.float64)) @ np.abs(h.dequant_f64()).T
    assert np.all(np.abs(yf - ref) <= 1e-5 * scale + 1e-30)
    assert _ulps_bf16(y, layout.f32_to_bf16(ref.astype(np.float32))).max() <= 1
    np.testing.assert_array_equal(y, layout.f32_to_bf16(yf))


@pytest.mark.parametrize("bits,gs", [(4, 64), (6, 64), (4, 32), (4, 128), (6, 128)])
def test_gemv_replays_chunk_order_exactly(orc, rng, bits, gs):
    n, k = 3, 256
    h = layout.synth_quant(rng, n, k, bits, group_size=gs)
    x = layout.synth_bf16(rng, (1, k))
    _, yf = orc.gemv_quant(h, x, 1, want_f32=True)
    q = layout.unpack_codes(h.codes, bits, k)
    xf = bf(x[0])
    for r in range(n):
        want = exact.replay_qrow(q[r], xf, bf(h.scales[r]), bf(h.biases[r]), gs)
        assert yf[0, r].view(np.uint32) == np.float32(want).view(np.uint32)


def test_gemv_replay_beyond_64_chunks(orc, rng):
    # K = 4096 -> 128 chunks: lanes sum two chunks each before the butterfly
    n, k = 2, 4096
    h = layout.synth_quant(rng, n, k, 4)
    x = layout.synth_bf16(rng, (1, k))
    _, yf = orc.gemv_quant(h, x, 1, want_f32=True)
    q = layout.unpack_codes(h.codes, 4, k)
    for r in range(n):
        want = exact.replay_qrow(q[r], bf(x[0]), bf(h.scales[r]), bf(h.biases[r]), 64)
        assert yf[0, r] == want


@pytest.mark.parametrize("bits", [4, 6])
def test_gemv_one_hot_reproduces_dequant(orc, rng, bits):
    # x = e_k: every chunk but one contributes +0 and the live chunk is
    # fma(s, q, b*1): one rounding, exactly the dequantized weight
    n, k = 32, 512
    h = layout.synth_quant(rng, n, k, bits)
    deq = orc.dequant_bf16(h)
    for col in (0, 1, 63, 64, 255, 511):
        x = np.zeros((1, k), np.uint16)
        x[0, col] = 0x3F80  # bf16 1.0
        y = orc.gemv_quant(h, x, 1)
        np.testing.assert_array_equal(y[0], deq[:, col])


def test_gemv_zero_codes_and_zero_scale(orc, rng):
    n, k = 8, 256
    h = layout.synth_quant(rng, n, k, 4)
    x = layout.synth_bf16(rng, (1, k))
    xs = bf(x[0]).astype(np.float64).reshape(-1, 64).sum(axis=1)
    for mode in ("codes", "scales"):
        hz = layout.HostQuant(h.codes.copy(), h.scales.copy(), h.biases.copy(), n, k, 64, 4)
        if mode == "codes":
            hz.codes[:] = 0
        else:
            hz.scales[:] = 0
        _, yf = orc.gemv_quant(hz, x, 1, want_f32=True)
        ref = bf(h.biases).astype(np.float64) @ xs
        np.testing.assert_allclose(yf[0], ref, rtol=1e-5, atol=1e-6)


def test_gemv_all_ones_is_row_sum(orc, rng):
    n, k = 16, 1024
    h = layout.synth_quant(rng, n, k, 6)
    x = np.full((1, k), 0x3F80, np.uint16)  # bf16 1.0
    _, yf = orc.gemv_quant(h, x, 1, want_f32=True)
    np.testing.assert_allclose(yf[0], h.dequant_f64().sum(axis=1), rtol=1e-5)


def test_gemv_rows_subset(orc, rng):
    h = layout.synth_quant(rng, 100, 512, 4)
    x = layout.synth_bf16(rng, (2, 512))
    y = orc.gemv_quant(h, x, 2)
    rows = np.array([0, 7, 99, 50], np.uint32)
    np.testing.assert_array_equal(orc.gemv_quant_rows(h, x, rows, 2), y[:, rows])


@pytest.mark.parametrize("bits", [4, 6, 8])
def test_dequant_is_one_rounding(orc, rng, bits):
    h = layout.synth_quant(rng, 16, 256, bits)
    deq = orc.dequant_bf16(h)
    q = layout.unpack_codes(h.codes, bits, 256).astype(np.float64)
    assert q.max() > (1 << (bits - 1))  # the codes reach the upper half of the range
    s = np.repeat(bf(h.scales), 64, axis=1).astype(np.float64)
    b = np.repeat(bf(h.biases), 64, axis=1).astype(np.float64)
    # s*q is exact in f64 (q < 256, 8-bit s); + b then one rounding to f32 is
    # the fma (f64 sum exact here), then RNE to bf16
    want = layout.f32_to_bf16((s * q + b).astype(np.float32))
    np.testing.assert_array_equal(deq, want)


@pytest.mark.parametrize("w_f32", [True, False])
def test_dense_gemv(orc, rng, w_f32):
    n, k, m = 64, 2048, 3
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    wd = w if w_f32 else layout.f32_to_bf16(w)
    x = layout.synth_bf16(rng, (m, k))
    y = orc.gemv_dense(wd, x)
    wf = w.astype(np.float64) if w_f32 else bf(wd).astype(np.float64)
    ref = bf(x).astype(np.float64) @ wf.T
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)
    # exact replay of two entries
    for t, e in ((0, 0), (2, 63)):
        want = exact.replay_dense_row(wf[e].astype(np.float32), bf(x[t]))
        assert y[t, e] == want


# ---- decode GEMV epilogue variants (lfm.metal:1023-1109) -------------------

def test_proj3_is_three_gemvs_and_a_cache_write(orc, rng):
    """Pins orc_proj3: q and k equal the GEMV rows; the V rows land at
    position pos of each 64-wide head of the cache (checked through a reshape,
    not the index formula) and nothing else in the cache changes."""
    k, nq, nk, nv, max_seq, pos = 512, 48, 16, 128, 6, 4
    hq, hk, hv = (layout.synth_quant(rng, n, k, 4) for n in (nq, nk, nv))
    x = layout.synth_bf16(rng, (1, k))[0]
    cache = np.full((nv // 64, max_seq, 64), 0x7fc1, np.uint16)
    q, kk = orc.proj3(hq, hk, hv, x, max_seq, pos, cache)
    np.testing.assert_array_equal(q, orc.gemv_quant(hq, x)[0])
    np.testing.assert_array_equal(kk, orc.gemv_quant(hk, x)[0])
    np.testing.assert_array_equal(cache[:, pos, :], orc.gemv_quant(hv, x)[0].reshape(nv // 64, 64))
    rest = np.delete(cache, pos, axis=1)
    assert (rest == 0x7fc1).all()


def _bf16_round(v):
    return layout.bf16_to_f32(layout.f32_to_bf16(np.asarray(v, np.float32)))


def test_conv3_reduces_to_its_inputs_for_one_hot_taps(orc, rng):
    """Pins orc_conv3's indexing: with taps (1, 0, 0) the conv output is
    bf16(C * state[c]); with (0, 0, 1) it is bf16(C * bf16(B X)); the state
    shifts (new_state[0] = state[1], new_state[1] = bf16(B X)); B, C, X are
    the GEMV row blocks 0, H, 2H."""
    H, k = 40, 512
    h = layout.synth_quant(rng, 3 * H, k, 4)
    x = layout.synth_bf16(rng, (1, k))[0]
    state = layout.synth_bf16(rng, (2, H))
    rows = layout.bf16_to_f32(orc.gemv_quant(h, x)[0])
    B, C, X = rows[:H], rows[H:2 * H], rows[2 * H:]
    bx = _bf16_round(B * X)
    one = layout.f32_to_bf16(np.float32(1.0))
    for hot, want in ((0, _bf16_round(C * layout.bf16_to_f32(state[0]))), (2, _bf16_round(C * bx))):
        taps = np.zeros((H, 3), np.uint16)
        taps[:, hot] = one
        out, ns = orc.conv3(h, x, taps, state)
        np.testing.assert_array_equal(layout.bf16_to_f32(out), want)
        np.testing.assert_array_equal(ns[0], state[1])
        np.testing.assert_array_equal(layout.bf16_to_f32(ns[1]), bx)


def test_conv3_taps_sum_in_order(orc, rng):
    """General taps: z = t0 s0 + t1 s1 + t2 v2 in f32, left to right."""
    H, k = 24, 256
    h = layout.synth_quant(rng, 3 * H, k, 4)
    x = layout.synth_bf16(rng, (1, k))[0]
    state = layout.synth_bf16(rng, (2, H))
    taps = layout.synth_bf16(rng, (H, 3), std=0.5)
    out, _ = orc.conv3(h, x, taps, state)
    rows = layout.bf16_to_f32(orc.gemv_quant(h, x)[0])
    t = layout.bf16_to_f32(taps)
    s = layout.bf16_to_f32(state)
    v2 = _bf16_round(rows[:H] * rows[2 * H:])
    z = (t[:, 0] * s[0] + t[:, 1] * s[1]).astype(np.float32) + (t[:, 2] * v2).astype(np.float32)
    np.testing.assert_array_equal(layout.bf16_to_f32(out), _bf16_round(rows[H:2 * H] * _bf16_round(z)))


# ---- token tail + Q6 embedding (lfm.metal:430-462, :1284-1386) ------------

def test_token_tail_embed_row_and_norm(orc, rng):
    """Pins orc_token_tail_embed: the token is the key's, the key is cleared,
    the row equals the dequant oracle's row, and the norm is within bf16
    rounding of float64 RMSNorm."""
    n, k, eps = 300, 2048, 1e-5
    h = layout.synth_quant(rng, n, k, 6)
    w = layout.synth_bf16(rng, (k,), std=0.3)
    tok = 217
    key = (0x9abc1234 << 32) | (~tok & 0xffffffff)
    got_tok, x, normed, after = orc.token_tail_embed(key, h, w, eps)
    assert got_tok == tok and after == 0
    np.testing.assert_array_equal(x, orc.dequant_bf16(h)[tok])
    xv = bf(x).astype(np.float64)
    ref = xv / np.sqrt(np.mean(xv * xv) + eps) * bf(w).astype(np.float64)
    got = bf(normed).astype(np.float64)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) <= 2.0 ** -7


def test_token_tail_embed_constant_row(orc):
    """A row of one value c: normed = bf16(c / sqrt(c^2 + eps) * w) (closed form)."""
    k, eps = 512, 1e-6
    q = np.full((1, k), 5, np.uint8)
    h = layout.HostQuant(codes=orc.pack(q.ravel(), 6).reshape(1, -1),
                         scales=layout.f32_to_bf16(np.full((1, k // 64), 0.25, np.float32)),
                         biases=layout.f32_to_bf16(np.full((1, k // 64), -2.0, np.float32)),
                         n=1, k=k, group_size=64, bits=6)
    w = layout.f32_to_bf16(np.linspace(-1, 1, k).astype(np.float32))
    _, x, normed, _ = orc.token_tail_embed(~0 & 0xffffffff, h, w, eps)  # token 0
    c = np.float32(0.25 * 5 - 2.0)
    assert (bf(x) == c).all()
    inv = np.float32(1.0) / np.sqrt(np.float32(c * c) + np.float32(eps), dtype=np.float32)
    np.testing.assert_array_equal(bf(normed), bf(layout.f32_to_bf16((c * inv) * bf(w))))
