"""GPU parity of the prefill MoE path through the C ABI.

Integer outputs (routing ids, counts, offsets, the stable sort, block maps)
are compared bit for bit.  Grouped-GEMM outputs accumulate in the MFMA's own
order, so they are compared to the oracle within tolerance: rel-L2 <= 5e-3
and max |err| <= 2e-2 x max|ref| (bf16 outputs of magnitude ~1e3 make an
absolute 2e-2 bar equivalent to bit-exactness)."""
import numpy as np
import pytest

from molten_amd import hip, layout
from tests.devutil import dev_quant, empty_dev, float_report, from_dev, to_dev, zeros_dev
from tests.synth import moe_weights, router_weights

pytestmark = pytest.mark.gpu
bf = layout.bf16_to_f32


def _log(msg):
    print(msg, flush=True)


def assert_close(got_bf16, ref_bf16, what, rel_l2=5e-3, max_rel=2e-2):
    """Tolerance of the float outputs: rel-L2 <= 5e-3 and max abs err <= 2e-2
    x max |ref|; the literal max abs err and the bf16-ulp histogram are
    printed (float_report)."""
    g = bf(got_bf16).astype(np.float64)
    r = bf(ref_bf16).astype(np.float64)
    l2 = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
    mx = np.abs(g - r).max() / max(np.abs(r).max(), 1e-30)
    float_report(got_bf16, ref_bf16, what)
    _log(f"{what}: rel-L2 {l2:.2e}, max|err|/max|ref| {mx:.2e}, "
         f"bit-equal {np.mean(got_bf16 == ref_bf16):.4f}")
    assert l2 <= rel_l2 and mx <= max_rel, (what, l2, mx)


def _routing(rng, m, e, topk, skew=None):
    if skew == "one":
        return np.tile(np.arange(topk, dtype=np.uint32), (m, 1))
    if skew == "sparse":
        pool = rng.choice(e, 5, replace=False)
        return np.stack([rng.choice(pool, topk, replace=False) for _ in range(m)]).astype(np.uint32)
    return np.stack([rng.choice(e, topk, replace=False) for _ in range(m)]).astype(np.uint32)


@pytest.mark.parametrize("skew", [None, "one", "sparse"])
@pytest.mark.parametrize("m", [4096, 37])
def test_counting_sort_bit_exact(dev, orc, m, skew):
    rng = np.random.default_rng(m)
    e, topk = 64, 4
    ids = _routing(rng, m, e, topk, skew)
    d_ids = to_dev(ids)
    counts = empty_dev((e,), np.uint32)
    offsets = empty_dev((e,), np.uint32)
    ids_sorted = empty_dev((m * topk,), np.uint32)
    slotpos = empty_dev((m * topk,), np.uint32)
    hip.moe_zero_counts(counts, e)
    hip.moe_count_slots(d_ids, counts, m * topk, e)
    hip.moe_offsets(counts, offsets, e)
    hip.moe_sorted(d_ids, offsets, ids_sorted, slotpos, m, e, topk)
    want_c = orc.moe_count(ids, e)
    want_o = orc.moe_offsets(want_c)
    want_s, want_p = orc.moe_sorted(ids, want_o, m, e, topk)
    np.testing.assert_array_equal(from_dev(counts, np.uint32), want_c)
    np.testing.assert_array_equal(from_dev(offsets, np.uint32), want_o)
    np.testing.assert_array_equal(from_dev(ids_sorted, np.uint32), want_s)
    np.testing.assert_array_equal(from_dev(slotpos, np.uint32), want_p)


@pytest.mark.parametrize("bm,gu_bn,dn_bn", [(128, 128, 256), (128, 64, 64), (32, 64, 64)])
def test_block_maps_bit_exact(dev, orc, bm, gu_bn, dn_bn):
    rng = np.random.default_rng(bm + gu_bn)
    m, e, topk, gu_n, dn_n = 4096, 64, 4, 1536, 2048
    ids = _routing(rng, m, e, topk, "sparse" if bm == 32 else None)
    counts = orc.moe_count(ids, e)
    offsets = orc.moe_offsets(counts)
    m_tiles = -(-m * topk // bm) + e
    max_gu, max_dn = m_tiles * gu_n // gu_bn, m_tiles * dn_n // dn_bn
    gu_off, dn_off = empty_dev((e,), np.uint32), empty_dev((e,), np.uint32)
    gu, dn = empty_dev((max_gu, 4), np.uint32), empty_dev((max_dn, 4), np.uint32)
    dc, do = to_dev(counts), to_dev(offsets)
    hip.moe_zero_blocks(gu, dn, max_gu, max_dn)
    hip.moe_block_offsets(dc, gu_off, dn_off, e, bm, gu_bn, dn_bn, gu_n, dn_n)
    hip.moe_blocks(dc, do, gu_off, dn_off, gu, max_gu, dn, max_dn, e, bm, gu_bn, dn_bn, gu_n, dn_n)
    w_go, w_do = orc.moe_block_offsets(counts, bm, gu_bn, dn_bn, gu_n, dn_n)
    w_gu, w_dn = orc.moe_blocks(counts, offsets, w_go, w_do, bm, gu_bn, dn_bn, gu_n, dn_n,
                                max_gu, max_dn)
    np.testing.assert_array_equal(from_dev(gu_off, np.uint32), w_go)
    np.testing.assert_array_equal(from_dev(dn_off, np.uint32), w_do)
    np.testing.assert_array_equal(from_dev(gu, np.uint32), w_gu)
    np.testing.assert_array_equal(from_dev(dn, np.uint32), w_dn)


def test_gather_silu_combine_bit_exact(dev, orc):
    rng = np.random.default_rng(5)
    m, h, topk = 333, 2048, 4
    table = layout.synth_bf16(rng, (m, h))
    ids = rng.integers(0, m, m * topk).astype(np.uint32)
    out = empty_dev((m * topk, h), np.uint16)
    hip.gather_rows_bf16(to_dev(table), to_dev(ids), out, m * topk, h, m)
    np.testing.assert_array_equal(from_dev(out, np.uint16), orc.gather_rows_bf16(table, ids))
    g = layout.synth_bf16(rng, (m, 1536), std=5.0)
    u = layout.synth_bf16(rng, (m, 1536), std=3.0)
    act = empty_dev((m, 1536), np.uint16)
    hip.silu_mul_bf16(to_dev(g), to_dev(u), act, g.size)
    np.testing.assert_array_equal(from_dev(act, np.uint16), orc.silu_mul_bf16(g, u))
    slotpos = rng.permutation(m * topk).astype(np.uint32)
    w = layout.synth_bf16(rng, (m, topk), std=0.3)
    comb = empty_dev((m, h), np.uint16)
    hip.moe_combine_rows(to_dev(table.repeat(topk, axis=0)), to_dev(slotpos), to_dev(w), comb, m,
                         h, topk)
    np.testing.assert_array_equal(from_dev(comb, np.uint16),
                                  orc.moe_combine_rows(table.repeat(topk, axis=0), slotpos, w, m,
                                                       topk))


def _map(orc, counts, bm, bn, n):
    offsets = orc.moe_offsets(counts)
    go, _ = orc.moe_block_offsets(counts, bm, bn, bn, n, n)
    s = int(counts.sum())
    max_e = (-(-s // bm) + counts.size) * (n // bn)
    gu, _ = orc.moe_blocks(counts, offsets, go, go, bm, bn, bn, n, n, max_e, max_e)
    return gu, max_e, offsets


@pytest.mark.parametrize("tile", [(512, 256), (256, 256), (128, 256), (128, 64), (32, 64)])
def test_grouped_gemm_one_hot_is_exact_dequant(dev, orc, tile):
    """A = unit rows: every output is one dequantized weight, so the in-register
    bf16(fma(s, q, b)) dequant must match the oracle's bit for bit."""
    bm, bn = tile
    rng = np.random.default_rng(bm + bn)
    e, n, k = 5, 512, 2048
    w = layout.synth_quant(rng, e * n, k, 4)
    # 300 rows: two balanced passes of the segment kernels (5 + 5 blocks);
    # 513: two map entries at bm = 512, one of a single row; 280: one pass of
    # 9 row blocks (the ninth block's accumulators in arch VGPRs)
    counts = np.array([40, 0, 300, 513, 280], np.uint32)
    s = int(counts.sum())
    cols = rng.integers(0, k, s)
    a = np.zeros((s, k), np.uint16)
    a[np.arange(s), cols] = 0x3F80
    blocks, max_e, offsets = _map(orc, counts, bm, bn, n)
    wd, keep = dev_quant(w)
    c = zeros_dev((s, n), np.uint16)
    hip.gemm_q4_grouped_mlx(to_dev(a), wd, c, to_dev(blocks), max_e, s, n, tile)
    deq = orc.dequant_bf16(w)
    got = from_dev(c, np.uint16)
    for ex in range(e):
        for i in range(offsets[ex], offsets[ex] + counts[ex]):
            np.testing.assert_array_equal(got[i], deq[ex * n:(ex + 1) * n, cols[i]])


@pytest.mark.parametrize("tile", [(512, 256), (256, 256), (128, 256), (128, 64), (32, 64)])
def test_grouped_gemm_vs_oracle(dev, orc, tile):
    rng = np.random.default_rng(7 + tile[0] + tile[1])
    e, n, k = 8, 1024, 1536
    w = layout.synth_quant(rng, e * n, k, 4)
    counts = rng.integers(0, 300, e).astype(np.uint32)
    counts[2] = 0
    counts[5] = 1
    counts[6] = 288  # nine full row blocks: one pass of the segment kernel
    s = int(counts.sum())
    a = layout.synth_bf16(rng, (s, k), std=3.0)
    blocks, max_e, _ = _map(orc, counts, tile[0], tile[1], n)
    wd, keep = dev_quant(w)
    c = zeros_dev((s, n), np.uint16)
    hip.gemm_q4_grouped_mlx(to_dev(a), wd, c, to_dev(blocks), max_e, s, n, tile)
    want = orc.gemm_q4_grouped(a, w, blocks, max_e, n, tile[1])
    assert_close(from_dev(c, np.uint16), want, f"grouped gemm {tile}")


@pytest.mark.parametrize("tile", [(512, 128), (256, 128), (128, 128), (128, 64), (32, 64)])
def test_grouped_gate_up_and_fused_act(dev, orc, tile):
    rng = np.random.default_rng(11 + tile[0] + tile[1])
    e, n, k, t = 6, 512, 2048, 300
    gate = layout.synth_quant(rng, e * n, k, 4)
    up = layout.synth_quant(rng, e * n, k, 4)
    x = layout.synth_bf16(rng, (t, k))
    # expert 3 gets exactly 270 rows (one 9-row-block pass of the segment
    # kernel), the others share the rest
    ids = rng.integers(0, e - 1, (t, 2)).astype(np.uint32)
    ids[ids >= 3] += 1
    ids[:270, 0] = 3
    counts = orc.moe_count(ids, e)
    offsets = orc.moe_offsets(counts)
    ids_sorted, _ = orc.moe_sorted(ids, offsets, t, e, 2)
    s = t * 2
    gx = x[ids_sorted]
    blocks, max_e, _ = _map(orc, counts, tile[0], tile[1], n)
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    db = to_dev(blocks)
    go, uo = zeros_dev((s, n), np.uint16), zeros_dev((s, n), np.uint16)
    hip.gemm_q4_grouped_mlx_gu(to_dev(gx), dg, du, go, uo, db, max_e, s, n, tile)
    want_g = orc.gemm_q4_grouped(gx, gate, blocks, max_e, n, tile[1])
    want_u = orc.gemm_q4_grouped(gx, up, blocks, max_e, n, tile[1])
    assert_close(from_dev(go, np.uint16), want_g, f"gate {tile}")
    assert_close(from_dev(uo, np.uint16), want_u, f"up {tile}")
    act = zeros_dev((s, n), np.uint16)
    hip.gemm_q4_grouped_gu_act(to_dev(x), to_dev(ids_sorted), t, dg, du, act, db, max_e, s, n, tile)
    assert_close(from_dev(act, np.uint16), orc.silu_mul_bf16(want_g, want_u), f"act {tile}")


def _run_prefill(orc, m, mode, seed, sample=None):
    rng = np.random.default_rng(seed)
    E, H, I, topk = 64, 2048, 1536, 4
    gate, up, down = moe_weights(rng, E, H, I)
    router = router_weights(rng, E, H, f32=(mode == 0))
    bias = rng.normal(0, 0.05, E).astype(np.float32) if mode == 0 else None
    x = layout.synth_bf16(rng, (m, H))
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    dd, kd = dev_quant(down)
    total, offs = hip.moe_prefill_workspace(m, E, topk, H, I)
    ws = zeros_dev((total // 4,), np.uint32)
    out = zeros_dev((m, H), np.uint16)
    hip.moe_prefill(to_dev(router), None if bias is None else to_dev(bias), dg, du, dd, E, topk,
                    to_dev(x), m, out, ws, total, mode=mode)
    mask = None
    if sample is not None:
        mask = np.zeros(m, np.uint8)
        mask[rng.choice(m, sample, replace=False)] = 1
    want = orc.moe_prefill(router, bias, mode, gate, up, down, E, topk, H, I, x, token_mask=mask)
    wsb = from_dev(ws, np.uint32).view(np.uint8)

    def region(name, dtype, count):
        o = offs[name]
        return wsb[o:o + count * np.dtype(dtype).itemsize].view(dtype)

    s = m * topk
    got = dict(ids=region("ids", np.uint32, s).reshape(m, topk),
               gw=region("gw", np.uint16, s).reshape(m, topk),
               counts=region("counts", np.uint32, E), offsets=region("offsets", np.uint32, E),
               ids_sorted=region("ids_sorted", np.uint32, s),
               slotpos=region("slotpos", np.uint32, s),
               out=from_dev(out, np.uint16))
    return got, want, mask


def _launch_order(ents, nt):
    """The segment GEMMs' launch order of a block map (CPU restatement of
    mh::seg_rank_of / seg_workgroup_of): map rows (nt entries each) ranked by
    row count, most first, lower row first on ties; rank r's column tile t at
    workgroup ((r // 8) * nt + t) * 8 + x, x = r % 8 on even r // 8 and
    7 - r % 8 on odd; the grid whole units of 8 x nt, other entries zero."""
    n_rows = len(ents) // nt
    counts = [int(ents[c * nt, 3]) - int(ents[c * nt, 0]) if ents[c * nt, 3] > ents[c * nt, 0] else 0
              for c in range(n_rows)]
    used = [c for c in range(n_rows) if counts[c] > 0]
    order = sorted(used, key=lambda c: (-counts[c], c))
    unit = 8 * nt
    grid = -(-len(ents) // unit) * unit
    out = np.zeros((grid, 4), np.uint32)
    for r, c in enumerate(order):
        slot, xr = divmod(r, 8)
        x = 7 - xr if slot & 1 else xr
        for t in range(nt):
            out[(slot * nt + t) * 8 + x] = ents[c * nt + t]
    return out


@pytest.mark.parametrize("skewed", [False, True])
def test_moe_prefill_stamped_matches_unstamped(dev, orc, skewed):
    """The prefill step's grouped GEMMs run on the block maps in launch order
    (gu_ord / dn_ord): those equal the CPU restatement of the order over the
    reference-order maps (gu_map / dn_map), and the GEMMs over them give the
    same bits as the public grouped GEMMs over the reference-order maps.  The
    measurement form (stamped per workgroup) gives the same bits as
    mh_moe_prefill; each GEMM's stamps form one prefix of workgroups, each
    with its start before its end, and the workgroups with rows are exactly
    the launch-ordered map's non-empty entries, with their row counts.  The
    launch-ordered grouped-GEMM entry points give the same bits too.
    Skewed: sigmoid + bias routing whose bias sends every token to experts 5,
    9 and 40 (1024 rows each: two map rows of 512, tied) and one other."""
    _log(f"moe prefill stamped m=1024 skewed={skewed}")
    rng = np.random.default_rng(77)
    E, H, I, topk, m = 64, 2048, 1536, 4, 1024
    gate, up, down = moe_weights(rng, E, H, I)
    router = router_weights(rng, E, H, f32=False)
    x = to_dev(layout.synth_bf16(rng, (m, H)))
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    dd, kd = dev_quant(down)
    bias, mode = None, 1
    if skewed:
        b = np.zeros(E, np.float32)
        b[[5, 9, 40]] = 1.0e4
        bias, mode = to_dev(b), 0
    total, offs = hip.moe_prefill_workspace(m, E, topk, H, I)
    outs, wss = [], []
    stamps = zeros_dev((2 * hip.PREFILL_STAMP_WGS * hip.PREFILL_STAMPS,), np.uint64)
    for stamped in (False, True):
        ws = zeros_dev((total // 4,), np.uint32)
        out = zeros_dev((m, H), np.uint16)
        r = to_dev(router)
        if stamped:
            hip.moe_prefill_stamped(r, bias, dg, du, dd, E, topk, x, m, out, ws, total, stamps, mode=mode)
        else:
            hip.moe_prefill(r, bias, dg, du, dd, E, topk, x, m, out, ws, total, mode=mode)
        outs.append(from_dev(out, np.uint16))
        wss.append(from_dev(ws, np.uint32).view(np.uint8))
    np.testing.assert_array_equal(outs[1], outs[0])
    np.testing.assert_array_equal(wss[1], wss[0])

    def region(key):
        o = offs[key]
        nxt = min([v for v in offs.values() if v > o] + [total])
        return wss[1][o:nxt].view(np.uint32).reshape(-1, 4)

    s = m * topk
    counts = region("counts").reshape(-1)[:E]
    if skewed:
        assert (counts[[5, 9, 40]] == m).all() and counts.sum() == s
    gu_nt, dn_nt = I // hip.MoeTile.GU512[1], H // hip.MoeTile.DN512[1]
    n_rows = -(-s // hip.MoeTile.GU512[0]) + E
    # the public GEMMs over the reference-order maps, on the step's own ids_sorted
    base = ws.data_ptr()
    act = zeros_dev((s, I), np.uint16)
    ed = zeros_dev((s, H), np.uint16)
    hip.gemm_q4_grouped_gu_act(x, base + offs["ids_sorted"], m, dg, du, act, base + offs["gu_map"],
                               n_rows * gu_nt, s, I, hip.MoeTile.GU512)
    hip.gemm_q4_grouped_mlx(base + offs["act"], dd, ed, base + offs["dn_map"], n_rows * dn_nt, s, H,
                            hip.MoeTile.DN512)
    np.testing.assert_array_equal(from_dev(act, np.uint16).reshape(-1), wss[1][offs["act"]:].view(np.uint16)[:s * I])
    np.testing.assert_array_equal(from_dev(ed, np.uint16).reshape(-1), wss[1][offs["ed"]:].view(np.uint16)[:s * H])
    # the launch-ordered entry points over the workspace's launch-ordered maps
    act.zero_()
    ed.zero_()
    hip.gemm_q4_grouped_gu_act_ordered(x, base + offs["ids_sorted"], m, dg, du, act, base + offs["gu_ord"],
                                       hip.map_grid(n_rows * gu_nt, gu_nt), s, I, hip.MoeTile.GU512)
    hip.gemm_q4_grouped_ordered(base + offs["act"], dd, ed, base + offs["dn_ord"], hip.map_grid(n_rows * dn_nt, dn_nt),
                                s, H, hip.MoeTile.DN512)
    np.testing.assert_array_equal(from_dev(act, np.uint16).reshape(-1), wss[1][offs["act"]:].view(np.uint16)[:s * I])
    np.testing.assert_array_equal(from_dev(ed, np.uint16).reshape(-1), wss[1][offs["ed"]:].view(np.uint16)[:s * H])

    st = from_dev(stamps, np.uint64).reshape(2, hip.PREFILL_STAMP_WGS, hip.PREFILL_STAMPS)
    for g, key, nt in ((0, "gu", gu_nt), (1, "dn", dn_nt)):
        ents = region(key + "_map")[:n_rows * nt]
        ordm = region(key + "_ord")
        want = _launch_order(ents, nt)
        np.testing.assert_array_equal(ordm[:len(want)], want, err_msg=key + "_ord")
        live = set(int(i) for i in np.nonzero(want[:, 3] > want[:, 0])[0])
        s_g = st[g]
        n_wg = int((s_g[:, 0] != 0).sum())
        assert n_wg == len(want) and (s_g[:n_wg, 0] != 0).all() and not s_g[n_wg:].any()
        assert (s_g[:n_wg, 1] >= s_g[:n_wg, 0]).all()
        named = (s_g[:n_wg, 2] & 0xffffffff).astype(np.int64)
        rows = (s_g[:n_wg, 2] >> 32).astype(np.int64)
        assert (named == np.arange(n_wg)).all()
        assert set(np.nonzero(rows > 0)[0].tolist()) == live
        assert (rows == (want[:, 3].astype(np.int64) - want[:, 0].astype(np.int64)).clip(0)).all()
        got_entry = s_g[:n_wg, 3]
        has = rows > 0
        assert (got_entry[~has] == 0).all()
        assert ((got_entry[has] >= s_g[:n_wg, 0][has]) & (got_entry[has] <= s_g[:n_wg, 1][has])).all()


@pytest.mark.parametrize("m", [256, 300])
@pytest.mark.parametrize("mode", [1, 0])
def test_moe_prefill_small(dev, orc, mode, m):
    """The whole step (routing, sort, launch-ordered maps, GEMMs, combine) at
    256 tokens and at 300 (a partial last routing block of 12 tokens)."""
    _log(f"moe prefill m={m} mode={mode}")
    got, want, _ = _run_prefill(orc, m, mode, 40 + mode + m)
    for key in ("ids", "gw", "counts", "offsets", "ids_sorted", "slotpos"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    assert_close(got["out"], want["out"], f"prefill out m={m} mode={mode}")


@pytest.mark.parametrize("mode", [1, 0])
def test_moe_prefill_config4_full_size(dev, orc, mode):
    """Config 4 (4096 tokens, top-4 of 64), softmax routing with a bf16 router
    and sigmoid + bias routing with an f32 router: routing, counts, offsets
    and the sort bit-exact over all 16384 slots; the output of every token
    against the oracle's expert GEMMs."""
    _log(f"moe prefill config 4 full size mode={mode}")
    got, want, _ = _run_prefill(orc, 4096, mode, 2026 + mode)
    for key in ("ids", "gw", "counts", "offsets", "ids_sorted", "slotpos"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    assert_close(got["out"], want["out"], f"prefill out config 4 mode={mode} (all 4096 tokens)")


@pytest.mark.parametrize("m,e,h,mode", [(300, 64, 2048, 1), (300, 64, 2048, 0), (4096, 64, 2048, 1),
                                         (200, 48, 1024, 1), (200, 32, 1024, 0)])
def test_moe_prefill_bf16_router_routing(dev, orc, m, e, h, mode):
    """mh_moe_prefill's routing with a bf16 router, including expert counts
    below 64 and K = 1024: ids and weights bit-exact against the oracle's
    chunk-order logits routed on the CPU, and the stored logit of every chosen
    expert equal to the oracle's bit for bit.  The router holds an exact
    duplicate row (equal logits: the lower expert wins) and a row one bf16 ulp
    from another (a near tie); x holds a zero token (64 equal logits) and one
    with an infinite element."""
    _log(f"bf16 router routing m={m} e={e} h={h} mode={mode}")
    rng = np.random.default_rng(7 + m + e + mode)
    topk, n_inter = 4, 512
    gate, up, down = moe_weights(rng, e, h, n_inter)
    r = layout.f32_to_bf16(rng.normal(0, 0.02, (e, h)).astype(np.float32))
    r[7] = r[3]
    r[11] = r[5]
    r[11, 17] += 1
    bias = rng.normal(0, 0.05, e).astype(np.float32) if mode == 0 else None
    x = layout.synth_bf16(rng, (m, h))
    x[5] = 0
    x[9, 100] = 0x7f80
    # a token of bf16 denormals (logits in the f32 subnormal range) and one
    # with a few denormal elements among normal ones
    x[3] = rng.integers(1, 0x80, h).astype(np.uint16) | (rng.integers(0, 2, h).astype(np.uint16) << 15)
    x[4, ::7] = rng.integers(1, 0x80, len(x[4, ::7])).astype(np.uint16)
    # one normal element of 2^-120 among denormals: the denormals carry a
    # part of every logit far above the bound's 2^-138, so a matrix core that
    # flushed them would leave the stored approximations outside the bound
    x[6] = rng.integers(1, 0x80, h).astype(np.uint16) | (rng.integers(0, 2, h).astype(np.uint16) << 15)
    x[6, 0] = 0x0380
    dg, _ = dev_quant(gate)
    du, _ = dev_quant(up)
    dd, _ = dev_quant(down)
    total, offs = hip.moe_prefill_workspace(m, e, topk, h, n_inter)
    ws = zeros_dev((total // 4,), np.uint32)
    out = zeros_dev((m, h), np.uint16)
    hip.moe_prefill(to_dev(r), None if bias is None else to_dev(bias), dg, du, dd, e, topk,
                    to_dev(x), m, out, ws, total, mode=mode)
    wsb = from_dev(ws, np.uint32).view(np.uint8)
    ids = wsb[offs["ids"]:offs["ids"] + m * topk * 4].view(np.uint32).reshape(m, topk)
    gw = wsb[offs["gw"]:offs["gw"] + m * topk * 2].view(np.uint16).reshape(m, topk)
    lg = wsb[offs["logits"]:offs["logits"] + m * e * 4].view(np.float32).reshape(m, e)
    z = orc.gemv_dense(r, x)
    want_ids, want_gw = orc.route(z, bias, topk, mode)
    np.testing.assert_array_equal(ids, want_ids, err_msg="ids")
    np.testing.assert_array_equal(gw, want_gw, err_msg="weights")
    rows = np.arange(m)[:, None]
    np.testing.assert_array_equal(lg[rows, ids].view(np.uint32), z[rows, ids].view(np.uint32),
                                  err_msg="chosen logits")
    # the logits not recomputed (the matrix-core router's, bf16 routers of
    # <= 64 experts) lie within its bound 2^-12 sum |x w| + 2^-138 of the
    # chunk-order values
    xf = layout.bf16_to_f32(x).astype(np.float64)
    rf = layout.bf16_to_f32(r).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        c = np.abs(xf) @ np.abs(rf).T
        err = np.abs(lg.astype(np.float64) - z.astype(np.float64))
    fin = np.isfinite(c) & np.isfinite(z)
    bad = fin & ~(err <= c * 2.0 ** -12 + 2.0 ** -138)
    assert not bad.any(), (np.argwhere(bad)[:5], err[bad][:5], c[bad][:5])


def _dense_map(m, n, bm=128, bn=64):
    """Block map of a dense product (one matrix): (m0, n0, n0, m_end) per tile."""
    ents = [(m0, n0, n0, min(m0 + bm, m)) for m0 in range(0, m, bm) for n0 in range(0, n, bn)]
    return np.array(ents, np.uint32).reshape(-1, 4), len(ents)


@pytest.mark.parametrize("m,n,k", [(300, 2048, 2048), (64, 576, 1024), (4096, 512, 2048)])
def test_dense_gemm_vs_oracle(dev, orc, m, n, k):
    """The prefill dense projection (dequant + bf16 GEMM fused) against the
    oracle's grouped GEMM over a dense map."""
    rng = np.random.default_rng(m + n)
    w = layout.synth_quant(rng, n, k, 4)
    a = layout.synth_bf16(rng, (m, k))
    wd, keep = dev_quant(w)
    c = zeros_dev((m, n), np.uint16)
    hip.gemm_q4_dense(to_dev(a), m, wd, c)
    blocks, nb = _dense_map(m, n)
    assert_close(from_dev(c, np.uint16), orc.gemm_q4_grouped(a, w, blocks, nb, n, 64), f"dense {m}x{n}x{k}")


def test_dense_gemm_one_hot_is_exact_dequant(dev, orc):
    """Rows of A that are one-hot (x = 1 at column j) give dequantized column j exactly."""
    rng = np.random.default_rng(3)
    m, n, k = 200, 512, 1024
    w = layout.synth_quant(rng, n, k, 4)
    cols = rng.integers(0, k, m)
    a = np.zeros((m, k), np.uint16)
    a[np.arange(m), cols] = layout.f32_to_bf16(np.float32(1.0))
    wd, keep = dev_quant(w)
    c = zeros_dev((m, n), np.uint16)
    hip.gemm_q4_dense(to_dev(a), m, wd, c)
    np.testing.assert_array_equal(from_dev(c, np.uint16), orc.dequant_bf16(w)[:, cols].T)


@pytest.mark.parametrize("m,n,k", [(1100, 13312, 512), (1100, 7936, 512)])
def test_dense_gemm_segment_path(dev, orc, m, n, k):
    """Shapes with >= 256 segment entries of 256 x 256 (13312 columns: 5 row
    segments, the last of 76 rows, x 52 column tiles) or, below that, of
    128 x 256 (7936 columns: 9 row segments, the last of 76 rows, x 31): the
    segment kernel in dense mode.  One-hot rows reproduce the dequantized
    columns exactly over every tile, and the first and the last (partial)
    row segments match the oracle within tolerance."""
    rng = np.random.default_rng(11)
    w = layout.synth_quant(rng, n, k, 4)
    wd, keep = dev_quant(w)
    cols = rng.integers(0, k, m)
    a1 = np.zeros((m, k), np.uint16)
    a1[np.arange(m), cols] = layout.f32_to_bf16(np.float32(1.0))
    c = zeros_dev((m, n), np.uint16)
    hip.gemm_q4_dense(to_dev(a1), m, wd, c)
    deq = orc.dequant_bf16(w)
    np.testing.assert_array_equal(from_dev(c, np.uint16), deq[:, cols].T)
    a = layout.synth_bf16(rng, (m, k))
    hip.gemm_q4_dense(to_dev(a), m, wd, c)
    got = from_dev(c, np.uint16)
    ents = [(m0, n0, n0, min(m0 + 128, m)) for m0 in (0, 128, 1024) for n0 in range(0, n, 64)]
    blocks = np.array(ents, np.uint32).reshape(-1, 4)
    want = orc.gemm_q4_grouped(a, w, blocks, len(ents), n, 64)
    rows = np.r_[0:256, 1024:m]
    assert_close(got[rows], want[rows], f"dense segment path {m}x{n}x{k}")
