"""GPU parity of the decode GEMV family through the C ABI (BASELINE configs
1, 2 and 5).  Batch 1 (and shapes outside the matrix-core kernel's limits)
follows the oracle's chunk order: logits bit for bit.  Batch 2..8 on the
matrix-core kernel sums in another order: logits within the stated
tolerance (rel-L2 <= 5e-3, max abs err <= 2e-2 * max |ref|) and, as that
kernel's own property, within one bf16 ulp plus 1e-4 * max |ref| of the
oracle; argmax ids are exact on every path."""
import numpy as np
import pytest
import torch

from molten_amd import hip, layout
from tests.devutil import dev_quant, empty_dev, float_report, from_dev, to_dev, zeros_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _mfma_path(n, k, batch, gs=64):
    """Shapes the batched matrix-core kernel takes (gemv_mfma.hip limits)."""
    return 2 <= batch <= 8 and gs == 64 and k % 512 == 0 and k <= 2048 and n % 16 == 0


def _bf16_ulp(v):
    """bf16 ulp at |v| (2^(e - 7)); the least normal's for zero and denormals."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_scratch(scratch, n, k, batch, launches):
    """The finisher's slots are left zero; the last word counts the
    finisher's launches (chunk-order and matrix-core kernels alike)."""
    sc = from_dev(scratch, np.uint64)
    assert not sc[:-1].any()
    assert int(sc[-1]) == launches


def assert_logits(got, want, n, k, batch, gs=64):
    if not _mfma_path(n, k, batch, gs):
        np.testing.assert_array_equal(got, want)
        return
    float_report(got, want, f"logits n={n} k={k} batch={batch}")
    g = layout.bf16_to_f32(got).astype(np.float64)
    w = layout.bf16_to_f32(want).astype(np.float64)
    assert np.isfinite(g).all()
    rel_l2 = np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30)
    assert rel_l2 <= 5e-3, rel_l2
    assert np.abs(g - w).max() <= 2e-2 * np.abs(w).max()
    # the kernel's own accuracy: one bf16 ulp plus f32 rounding of the sums
    # (relative to the largest logit: cancellation near zero)
    assert (np.abs(g - w) <= _bf16_ulp(w) + 1e-4 * np.abs(w).max()).all()


@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("n,k,batch", [
    (2048, 2048, 1),   # config 1 shape
    (1536, 2048, 1),   # expert gate/up shape
    (2048, 1536, 1),   # expert down shape (48 live lanes)
    (300, 2048, 1),    # ragged last row group
    (1030, 2048, 1),   # two-wave workgroups (one to four 4-row blocks per CU), a partial last block
    (2050, 1536, 1),   # the same below K = 2048 (48 live lanes), partial last block
    (96, 11776, 1),    # dense down width: split-K path
    (2048, 11776, 1),  # the dense FFN down projection
    (37, 4160, 1),     # split-K: ragged rows, 130 chunks (a partial slab)
    (512, 2048, 2),
    (512, 2048, 8),    # config 5 batch
    (130, 1536, 5),
])
def test_gemv_matches_oracle(dev, orc, bits, n, k, batch):
    _log(f"gemv bits={bits} n={n} k={k} batch={batch}")
    rng = np.random.default_rng(n * 131 + k + batch + bits)
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    want = orc.gemv_quant(h, x, batch)
    w, keep = dev_quant(h)
    xd = to_dev(x)
    y = empty_dev((batch, n), np.uint16)
    hip.gemv_quant(w, xd, y, batch)
    got = from_dev(y, np.uint16)
    assert_logits(got, want, n, k, batch)


def _extreme_x(rng, batch, k, huge):
    """N(0,1) activations with f32-denormal, zero and -0 entries, and (huge)
    a few finite entries of magnitude 2^110."""
    x = rng.normal(0, 1, (batch, k)).astype(np.float32)
    idx = rng.choice(k, 64, replace=False)
    x[:, idx[:16]] = np.float32(2.0 ** -130) * np.sign(rng.normal(size=16)).astype(np.float32)
    x[:, idx[16:24]] = 0.0
    x[:, idx[24:32]] = -0.0
    if huge:
        x[:, idx[32:36]] = np.float32(2.0 ** 110) * np.array([1, -1, 1, -1], np.float32)
    return layout.f32_to_bf16(x)


@pytest.mark.parametrize("huge", [False, True])
@pytest.mark.parametrize("n,k,batch", [(512, 2048, 1), (96, 11776, 1), (256, 2048, 4)])
def test_q4_extreme_activations(dev, orc, huge, n, k, batch):
    """Denormal, signed-zero and (huge) 2^110 activations: the chunk-order
    kernels stay bit-exact; the matrix-core kernel (batch 4 here) stays within
    tolerance."""
    _log(f"q4 extreme x huge={huge} n={n} k={k} batch={batch}")
    rng = np.random.default_rng(5 + huge + k + batch)
    h = layout.synth_quant(rng, n, k, 4)
    x = _extreme_x(rng, batch, k, huge)
    want = orc.gemv_quant(h, x, batch)
    assert np.isfinite(layout.bf16_to_f32(want)).all()
    w, keep = dev_quant(h)
    y = empty_dev((batch, n), np.uint16)
    hip.gemv_quant(w, to_dev(x), y, batch)
    assert_logits(from_dev(y, np.uint16), want, n, k, batch)


@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("gs", [32, 128])
def test_gemv_other_group_sizes(dev, orc, bits, gs):
    rng = np.random.default_rng(gs + bits)
    h = layout.synth_quant(rng, 256, 2048, bits, group_size=gs)
    x = layout.synth_bf16(rng, (1, 2048))
    w, keep = dev_quant(h)
    y = empty_dev((1, 256), np.uint16)
    hip.gemv_quant(w, to_dev(x), y, 1)
    np.testing.assert_array_equal(from_dev(y, np.uint16), orc.gemv_quant(h, x, 1))


@pytest.mark.parametrize("bits,batch", [(4, 1), (6, 1), (6, 8), (4, 3)])
def test_argmax_paths_agree_with_oracle(dev, orc, bits, batch):
    _log(f"argmax bits={bits} batch={batch}")
    rng = np.random.default_rng(77 + bits * 10 + batch)
    n, k = 4096, 2048
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    logits = orc.gemv_quant(h, x, batch)
    want = [orc.argmax_bf16(logits[b]) for b in range(batch)]
    w, keep = dev_quant(h)
    xd = to_dev(x)
    # (1) stored logits + finisher ids, run twice to check the scratch is re-zeroed
    y = empty_dev((batch, n), np.uint16)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    ids = empty_dev((batch,), np.uint32)
    for call in range(3):
        hip.gemv_quant_argmax(w, xd, y, scratch, ids, batch)
        assert from_dev(ids, np.uint32).tolist() == want
        assert_scratch(scratch, n, k, batch, call + 1)
    assert_logits(from_dev(y, np.uint16), logits, n, k, batch)
    # (2) reference pair: head argmax (no logits) + token tail
    best = zeros_dev((batch,), np.uint64)
    tok = empty_dev((batch,), np.uint32)
    hip.gemv_head_argmax(w, xd, best, batch)
    hip.token_tail(best, tok, batch)
    assert from_dev(tok, np.uint32).tolist() == want
    assert from_dev(best, np.uint64).tolist() == [0] * batch


def test_lm_head_argmax_graph_replays(dev, orc):
    """The GEMV + argmax finisher captured in a HIP graph (three weight sets
    sharing one scratch) and replayed several times, with eager launches on
    the same scratch and cleared outputs between replays: every replay
    reproduces the eager logits and ids."""
    _log("graph replay gemv_quant_argmax")
    rng = np.random.default_rng(606)
    n, k = 8192, 2048
    hs = [layout.synth_quant(rng, n, k, 4) for _ in range(3)]
    x = layout.synth_bf16(rng, (1, k))
    devw = [dev_quant(h) for h in hs]
    xd = to_dev(x)
    want = [orc.gemv_quant(h, x, 1) for h in hs]
    want_ids = [orc.argmax_bf16(w[0]) for w in want]
    scratch = zeros_dev((hip.argmax_scratch_words(1),), np.uint64)
    ys = [empty_dev((1, n), np.uint16) for _ in hs]
    ids = [empty_dev((1,), np.uint32) for _ in hs]
    for (w, _), y, i in zip(devw, ys, ids):  # eager warm-up
        hip.gemv_quant_argmax(w, xd, y, scratch, i, 1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for (w, _), y, i in zip(devw, ys, ids):
            hip.gemv_quant_argmax(w, xd, y, scratch, i, 1)
    other_y = empty_dev((1, n), np.uint16)
    other_id = empty_dev((1,), np.uint32)
    launches = 3  # the eager warm-up calls (capture runs nothing)
    for rep in range(4):
        for y, i in zip(ys, ids):
            y.zero_()
            i.zero_()
        graph.replay()
        torch.cuda.synchronize()
        launches += 3
        for c in range(3):
            np.testing.assert_array_equal(from_dev(ys[c], np.uint16), want[c])
            assert int(from_dev(ids[c], np.uint32)[0]) == want_ids[c]
        assert_scratch(scratch, n, k, 1, launches)
        launches += 1
        hip.gemv_quant_argmax(devw[rep % 3][0], xd, other_y, scratch, other_id, 1)  # eager, same scratch
        torch.cuda.synchronize()
        assert int(from_dev(other_id, np.uint32)[0]) == want_ids[rep % 3]


def test_argmax_ignores_keys_of_earlier_launches(dev, orc):
    """A key that a late unit of an earlier launch left in its slot (planted
    here from the host: the largest possible key, tagged with the previous
    launch's tag) is never taken for this launch's: the ids stay the
    oracle's, the slot is re-zeroed and no wait expired."""
    rng = np.random.default_rng(4242)
    n, k = 8192, 2048
    h = layout.synth_quant(rng, n, k, 4)
    x = layout.synth_bf16(rng, (1, k))
    want = orc.argmax_bf16(orc.gemv_quant(h, x, 1)[0])
    w, keep = dev_quant(h)
    xd = to_dev(x)
    scratch = zeros_dev((hip.argmax_scratch_words(1),), np.uint64)
    ids = empty_dev((1,), np.uint32)
    hip.device_status(clear=True)
    for launch in range(3):
        sc = from_dev(scratch, np.uint64).copy()
        assert int(sc[-1]) == launch
        if launch > 0:
            stale_tag = (launch - 1) % 0xFFFF + 1
            sc[5] = np.uint64((stale_tag << 48) | 0xFFFFFFFFFFFF)
            scratch.copy_(to_dev(sc))
        hip.gemv_quant_argmax(w, xd, None, scratch, ids, 1)
        assert int(from_dev(ids, np.uint32)[0]) == want
        assert_scratch(scratch, n, k, 1, launch + 1)
    assert hip.device_status(clear=True) == 0


@pytest.mark.parametrize("bits,batch", [(4, 1), (6, 1), (4, 8)])
def test_argmax_after_expired_wait_is_reported(dev, orc, bits, batch):
    """The state an expired collector wait leaves (planted from the host): a
    slot word carrying the *current* launch's tag with the largest key (what
    a workgroup that started only after that collector gave up publishes)
    and bit 63 of the count word.  Such a word cannot be told from a fresh
    one, so the launch reports its result lost: ids 0xffffffff and
    MH_STATUS_ARGMAX_WAIT; it leaves the slots zero and the count advanced
    with the bit cleared, and the next launch is exact again."""
    _log(f"argmax after expired wait bits={bits} batch={batch}")
    rng = np.random.default_rng(4545 + bits + batch)
    n, k = 65536 if batch > 1 else 8192, 2048
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    want = [orc.argmax_bf16(row) for row in orc.gemv_quant(h, x, batch)]
    w, keep = dev_quant(h)
    xd = to_dev(x)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    ids = empty_dev((batch,), np.uint32)
    hip.device_status(clear=True)
    hip.gemv_quant_argmax(w, xd, None, scratch, ids, batch)
    assert from_dev(ids, np.uint32).tolist() == want
    sc = from_dev(scratch, np.uint64).copy()
    assert int(sc[-1]) == 1
    if batch == 1:
        # chunk-order finisher: tag of count 1, the largest 48-bit key, slot 5
        sc[5] = np.uint64((((1 % 0xFFFF) + 1) << 48) | 0xFFFFFFFFFFFF)
    else:
        # matrix-core finisher: workgroup 7's lower bound, the greatest finite
        # value under count 1's tag, in every batch row
        for r in range(batch):
            sc[r * hip.ARGMAX_SLOTS + 7] = ((np.uint64(0xFF7F0000) << np.uint64(32)) |
                                            (np.uint64(1 % 255 + 1) << np.uint64(24)) | np.uint64(0xFFFFFF))
    sc[-1] = np.uint64(1) | np.uint64(1 << 63)
    scratch.copy_(to_dev(sc))
    hip.gemv_quant_argmax(w, xd, None, scratch, ids, batch)
    assert from_dev(ids, np.uint32).tolist() == [0xFFFFFFFF] * batch
    assert hip.device_status(clear=True) & hip.STATUS_ARGMAX_WAIT
    assert_scratch(scratch, n, k, batch, 2)
    hip.gemv_quant_argmax(w, xd, None, scratch, ids, batch)
    assert from_dev(ids, np.uint32).tolist() == want
    assert_scratch(scratch, n, k, batch, 3)
    assert hip.device_status(clear=True) == 0


def test_mfma_argmax_ignores_untagged_words(dev, orc):
    """The matrix-core finisher takes only words with its launch's tag.
    Before each launch every slot of every batch row is filled from the host
    with words that would decide the argmax if taken (the greatest lower
    bound and candidates of the wrong rows): before the first launch random
    words whose tag is not 1, before the next ones the previous launch's tag.
    The finisher reads some slots before their workgroup publishes, so it
    meets the planted words; the ids stay the oracle's, the slots are left
    zero and the launch count advances."""
    rng = np.random.default_rng(4343)
    n, k, batch = 65536, 2048, 8
    h = layout.synth_quant(rng, n, k, 4)
    x = layout.synth_bf16(rng, (batch, k))
    want = [orc.argmax_bf16(row) for row in orc.gemv_quant(h, x, batch)]
    w, keep = dev_quant(h)
    xd = to_dev(x)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    ids = empty_dev((batch,), np.uint32)
    hip.device_status(clear=True)
    # the slots the finisher reads: word j of workgroup g (< 255) of batch
    # row r at r * ARGMAX_SLOTS + 256 j + g, six words per workgroup
    used = np.array([r * hip.ARGMAX_SLOTS + 256 * j + g for r in range(batch) for j in range(6)
                     for g in range(255)])
    for launch in range(3):
        sc = from_dev(scratch, np.uint64).copy()
        assert int(sc[-1]) == launch
        if launch == 0:
            junk = rng.integers(0, 2**63, used.size, dtype=np.uint64)
            tags = (junk >> np.uint64(24)) & np.uint64(0xFF)
            junk[tags == 1] ^= np.uint64(1 << 25)  # never this launch's tag
            sc[used] = junk
        else:
            # the greatest finite value, the previous launch's tag, row 65535
            stale = np.uint64((launch - 1) % 255 + 1)
            sc[used] = (np.uint64(0xFF7F0000) << np.uint64(32)) | (stale << np.uint64(24)) | np.uint64(0xFF0000)
        scratch.copy_(to_dev(sc))
        hip.gemv_quant_argmax(w, xd, None, scratch, ids, batch)
        assert [int(v) for v in from_dev(ids, np.uint32)] == want
        assert_scratch(scratch, n, k, batch, launch + 1)
    assert hip.device_status(clear=True) == 0


def test_argmax_ties_take_lowest_index(dev, orc):
    # identical rows -> identical logits: the lowest row must win
    rng = np.random.default_rng(5)
    h = layout.synth_quant(rng, 8, 2048, 4)
    rep = 700
    hb = layout.HostQuant(np.tile(h.codes[3:4], (rep, 1)), np.tile(h.scales[3:4], (rep, 1)),
                          np.tile(h.biases[3:4], (rep, 1)), rep, 2048, 64, 4)
    # make rows 0..99 smaller by zeroing their codes
    hb.codes[:100] = 0
    x = layout.synth_bf16(rng, (1, 2048))
    logits = orc.gemv_quant(hb, x, 1)[0]
    want = orc.argmax_bf16(logits)
    w, keep = dev_quant(hb)
    scratch = zeros_dev((hip.argmax_scratch_words(1),), np.uint64)
    ids = empty_dev((1,), np.uint32)
    hip.gemv_quant_argmax(w, to_dev(x), None, scratch, ids, 1)
    assert from_dev(ids, np.uint32)[0] == want


def test_two_stage_argmax(dev, orc):
    rng = np.random.default_rng(9)
    for n in (1, 63, 64, 1000, 65536, 128000):
        x = layout.synth_bf16(rng, (n,))
        if n > 10:
            x[n // 3] = x[n // 2] = layout.f32_to_bf16(np.float32([50.0]))[0]
        partials = empty_dev((64 * 2,), np.uint32)
        out = empty_dev((1,), np.uint32)
        hip.argmax_bf16(to_dev(x), n, partials, out)
        assert from_dev(out, np.uint32)[0] == orc.argmax_bf16(x)


@pytest.mark.parametrize("bits", [4, 6])
def test_dequant_bit_exact(dev, orc, bits):
    rng = np.random.default_rng(bits)
    h = layout.synth_quant(rng, 96, 2048, bits)
    w, keep = dev_quant(h)
    out = empty_dev((96, 2048), np.uint16)
    hip.dequant_to_bf16(w, out)
    np.testing.assert_array_equal(from_dev(out, np.uint16), orc.dequant_bf16(h))
    if bits == 4:
        out.zero_()
        hip.dequant_q4_bf16_bulk(w, out)
        np.testing.assert_array_equal(from_dev(out, np.uint16), orc.dequant_bf16(h))


@pytest.mark.parametrize("bits,batch", [(4, 1), (6, 1), (6, 8)])
def test_lm_head_full_size(dev, orc, bits, batch):
    """Configs 2 and 5 at their full 65536 x 2048 shape: logits against the
    oracle (bit-exact at batch 1, within tolerance at batch 8) and the ids
    are the oracle's argmax."""
    _log(f"lm head full bits={bits} batch={batch}")
    rng = np.random.default_rng(2026 + bits + batch)
    n, k = 65536, 2048
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    w, keep = dev_quant(h)
    y = empty_dev((batch, n), np.uint16)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    ids = empty_dev((batch,), np.uint32)
    hip.gemv_quant_argmax(w, to_dev(x), y, scratch, ids, batch)
    got = from_dev(y, np.uint16)
    got_ids = from_dev(ids, np.uint32)
    want = orc.gemv_quant(h, x, batch)
    assert_logits(got, want, n, k, batch)
    assert got_ids.tolist() == [orc.argmax_bf16(want[b]) for b in range(batch)]


@pytest.mark.parametrize("bits", [4, 6])
def test_stamped_head_matches_oracle(dev, orc, bits):
    """The measurement instantiation of the batch-1 head (phase timestamps)
    computes what the product kernel does: logits bit-exact, the oracle's id,
    the scratch re-zeroed and counted; every wave of the launch stamps its
    phases in order, wave 0 of every workgroup but the last publishes, and
    only the last workgroup's waves stamp the collection."""
    _log(f"stamped head bits={bits}")
    rng = np.random.default_rng(4242 + bits)
    n, k = 32768, 2048
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (1, k))
    w, keep = dev_quant(h)
    want = orc.gemv_quant(h, x, 1)
    y = empty_dev((1, n), np.uint16)
    scratch = zeros_dev((hip.argmax_scratch_words(1),), np.uint64)
    ids = empty_dev((1,), np.uint32)
    stamps = zeros_dev((hip.GEMV_STAMP_WAVES * hip.GEMV_STAMPS,), np.uint64)
    for call in range(2):
        hip.gemv_quant_argmax_stamped(w, to_dev(x), y, scratch, ids, stamps, 1)
        np.testing.assert_array_equal(from_dev(y, np.uint16), want)
        assert from_dev(ids, np.uint32).tolist() == [orc.argmax_bf16(want[0])]
        assert_scratch(scratch, n, k, 1, call + 1)
    st = from_dev(stamps, np.uint64).reshape(hip.GEMV_STAMP_WAVES, hip.GEMV_STAMPS).astype(np.int64)
    waves = n // 8  # one 8-row block per wave
    assert not st[waves:].any()
    st = st[:waves]
    assert (st[:, :5] > 0).all()
    assert (np.diff(st[:, :5], axis=1) >= 0).all()
    wg = np.arange(waves) // 4
    last = wg == wg.max()
    pub = (np.arange(waves) % 4 == 0) & ~last
    assert (st[pub, 5] >= st[pub, 4]).all() and not st[~pub, 5].any()
    assert (st[last, 6] >= st[last, 4]).all() and not st[~last, 6].any()
    assert (st[:, 7] < 16).all()


@pytest.mark.parametrize("bits", [4, 6])
def test_stamped_batch8_head_matches_oracle(dev, orc, bits):
    """The measurement instantiation of the batch-8 matrix-core head: ids the
    oracle's, logits within the kernel's tolerance, the scratch re-zeroed and
    counted; every wave of the 256 x 8 launch stamps its start, x staging and
    main loop in order, waves 0..7 of every workgroup their summary, and only
    the last workgroup's waves 0..7 the finisher's two phases and their count
    of recomputed rows."""
    _log(f"stamped batch-8 head bits={bits}")
    rng = np.random.default_rng(4343 + bits)
    n, k, batch = 8192, 2048, 8
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    w, keep = dev_quant(h)
    want = orc.gemv_quant(h, x, batch)
    y = empty_dev((batch, n), np.uint16)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    ids = empty_dev((batch,), np.uint32)
    stamps = zeros_dev((hip.GEMV_STAMP_WAVES * hip.GEMV_STAMPS,), np.uint64)
    for call in range(2):
        hip.gemv_quant_argmax_stamped(w, to_dev(x), y, scratch, ids, stamps, batch)
        assert from_dev(ids, np.uint32).tolist() == [orc.argmax_bf16(want[b]) for b in range(batch)]
        assert_scratch(scratch, n, k, batch, call + 1)
    assert_logits(from_dev(y, np.uint16), want, n, k, batch)
    st = from_dev(stamps, np.uint64).reshape(hip.GEMV_STAMP_WAVES, hip.GEMV_STAMPS).astype(np.int64)
    waves = 256 * 8
    assert not st[waves:].any()
    st = st[:waves]
    assert (st[:, :3] > 0).all() and (np.diff(st[:, :3], axis=1) >= 0).all()
    wave = np.arange(waves) % 8
    last = np.arange(waves) // 8 == 255
    assert (st[:, 3] >= st[:, 2]).all()
    assert (st[:, 4:6] > 0).all(axis=1).tolist() == last.tolist()
    assert (st[last, 5] >= st[last, 4]).all() and (st[last, 4] >= st[last, 3]).all()
    assert (st[:, 7] < 16).all()
    # word 6: the finisher waves' count of rows recomputed in chunk order
    assert not st[~last, 6].any() and (st[last, 6] <= n).all()


def _argmax_case(dev, orc, h, x, batch):
    w, keep = dev_quant(h)
    logits = orc.gemv_quant(h, x, batch)
    want = [orc.argmax_bf16(logits[b]) for b in range(batch)]
    y = empty_dev((batch, h.n), np.uint16)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    ids = empty_dev((batch,), np.uint32)
    for call in range(2):
        hip.gemv_quant_argmax(w, to_dev(x), y, scratch, ids, batch)
        assert from_dev(ids, np.uint32).tolist() == want
        assert_scratch(scratch, h.n, h.k, batch, call + 1)
    assert_logits(from_dev(y, np.uint16), logits, h.n, h.k, batch)
    return want


@pytest.mark.parametrize("bits", [4, 6])
def test_mfma_argmax_exact_ties(dev, orc, bits):
    """Matrix-core argmax with exact ties: the winning row copied to a lower
    and a higher index (equal bounds, so the finisher recomputes every row
    in chunk order); the lowest index must win."""
    _log(f"mfma argmax ties bits={bits}")
    rng = np.random.default_rng(313 + bits)
    n, k, batch = 2048, 2048, 3
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    top = orc.argmax_bf16(orc.gemv_quant(h, x, batch)[0])
    for dst in (5, min(n - 1, top + 700)):
        h.codes[dst] = h.codes[top]
        h.scales[dst] = h.scales[top]
        h.biases[dst] = h.biases[top]
    want = _argmax_case(dev, orc, h, x, batch)
    assert want[0] == min(5, top)


@pytest.mark.parametrize("bits", [4, 6])
def test_mfma_argmax_near_ties(dev, orc, bits):
    """Rows that differ from the winner in one code: values apart by one
    scale times one activation, often the same bf16 value, decided only by
    the chunk-order recomputation of the candidates."""
    _log(f"mfma argmax near ties bits={bits}")
    rng = np.random.default_rng(919 + bits)
    n, k, batch = 4096, 2048, 2
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    top = orc.argmax_bf16(orc.gemv_quant(h, x, batch)[1])
    words = h.codes.shape[1]
    for j, dst in enumerate((3, 1000, 2047, 4095)):
        if dst == top:
            continue
        h.codes[dst] = h.codes[top]
        h.scales[dst] = h.scales[top]
        h.biases[dst] = h.biases[top]
        h.codes[dst, (7 * j + 1) % words] ^= np.uint32(1 << (3 * j))
    _argmax_case(dev, orc, h, x, batch)


@pytest.mark.parametrize("pattern", [0xC7800000, 0x00000000])
def test_mfma_argmax_after_lds_garbage(dev, orc, pattern):
    """The matrix-core head after a kernel that left every CU's LDS holding
    one word pattern (-65536.0f or 0): its error bound uses the staged sum
    |x| of each batch row, which must be read after it is staged, never the
    LDS an earlier kernel left (a sum of -65536 turns every interval inside
    out: no candidate reaches the lower bound and every id comes out 0).
    Ids are the oracle's, logits within tolerance."""
    import ctypes
    import os

    import torch

    _log(f"mfma argmax after LDS fill {pattern:#010x}")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    lib = ctypes.CDLL(os.path.join(root, "molten_amd", "libmolten_ceiling.so"))
    lib.mhc_lds_fill.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    rng = np.random.default_rng(1701 + pattern % 7)
    n, k, batch = 16384, 2048, 8
    h = layout.synth_quant(rng, n, k, 6)
    x = layout.synth_bf16(rng, (batch, k))
    w, keep = dev_quant(h)
    want = orc.gemv_quant(h, x, batch)
    y = empty_dev((batch, n), np.uint16)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    ids = empty_dev((batch,), np.uint32)
    xd = to_dev(x)
    for call in range(2):
        assert lib.mhc_lds_fill(pattern, 4 * 256, torch.cuda.current_stream().cuda_stream) == 0
        hip.gemv_quant_argmax(w, xd, y, scratch, ids, batch)
        got_ids = from_dev(ids, np.uint32)
        assert got_ids.tolist() == [orc.argmax_bf16(want[b]) for b in range(batch)], call
    assert_logits(from_dev(y, np.uint16), want, n, k, batch)


@pytest.mark.parametrize("bits", [6, 4])
@pytest.mark.parametrize("tie", [False, True])
def test_model_head_128000_rows(dev, orc, tie, bits):
    """The reference model's own LM head: Q6 128000 x 2048 at batch 1
    (vocab 128000, src/lfm.rs:22-42, through gemv_head_argmax,
    src/kernels/lfm.rs:826-844), past the 65536 rows of the BASELINE configs;
    bits 4 runs the same rows through the Q4 head instantiation (held to five
    workgroups per CU).  Both entry points: mh_gemv_quant_argmax (logits
    bit-exact, id) and the reference pair mh_gemv_head_argmax +
    mh_token_tail.  With `tie` the winning row is copied to rows 65535 and
    65536 and to row 127999 (the rows on both sides of the 65536-row boundary
    and the last row), and the original winner is made smaller: the lowest
    copy, 65535, must win."""
    _log(f"model head 128000x2048 q{bits} tie={tie}")
    rng = np.random.default_rng(128000 + tie + 10 * bits)
    n, k = 128000, 2048
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (1, k))
    if tie:
        top = orc.argmax_bf16(orc.gemv_quant(h, x, 1)[0])
        for dst in (65535, 65536, 127999):
            h.codes[dst] = h.codes[top]
            h.scales[dst] = h.scales[top]
            h.biases[dst] = h.biases[top]
        if top not in (65535, 65536, 127999):
            h.codes[top] = 0
    logits = orc.gemv_quant(h, x, 1)
    want = orc.argmax_bf16(logits[0])
    if tie:
        assert want == 65535
    w, keep = dev_quant(h)
    xd = to_dev(x)
    y = empty_dev((1, n), np.uint16)
    scratch = zeros_dev((hip.argmax_scratch_words(1),), np.uint64)
    ids = empty_dev((1,), np.uint32)
    for call in range(2):
        hip.gemv_quant_argmax(w, xd, y, scratch, ids, 1)
        assert int(from_dev(ids, np.uint32)[0]) == want
        assert_scratch(scratch, n, k, 1, call + 1)
    assert_logits(from_dev(y, np.uint16), logits, n, k, 1)
    best = zeros_dev((1,), np.uint64)
    tok = empty_dev((1,), np.uint32)
    hip.gemv_head_argmax(w, xd, best, 1)
    hip.token_tail(best, tok, 1)
    assert int(from_dev(tok, np.uint32)[0]) == want
    assert int(from_dev(best, np.uint64)[0]) == 0
