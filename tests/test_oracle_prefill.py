"""Pins the oracle's prefill half: counting sort (a13), block maps (a14),
gather / SwiGLU / combine (a15, a17, a18), grouped GEMM (a16) and the step
composition (a19)."""
import numpy as np
import pytest

from molten_amd import layout
from tests.synth import moe_weights, router_weights

bf = layout.bf16_to_f32


def _routing(rng, m, e, topk, skew=None):
    if skew == "one":
        ids = np.tile(np.arange(topk, dtype=np.uint32), (m, 1))
    elif skew == "sparse":  # only 5 of e experts used
        pool = rng.choice(e, 5, replace=False)
        ids = np.stack([rng.choice(pool, topk, replace=False) for _ in range(m)]).astype(np.uint32)
    else:
        ids = np.stack([rng.choice(e, topk, replace=False) for _ in range(m)]).astype(np.uint32)
    return ids


@pytest.mark.parametrize("skew", [None, "one", "sparse"])
def test_counting_sort_matches_stable_argsort(orc, rng, skew):
    m, e, topk = 777, 64, 4
    ids = _routing(rng, m, e, topk, skew)
    counts = orc.moe_count(ids, e)
    np.testing.assert_array_equal(counts, np.bincount(ids.ravel(), minlength=e))
    offsets = orc.moe_offsets(counts)
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)[:-1]]))
    ids_sorted, slotpos = orc.moe_sorted(ids, offsets, m, e, topk)
    order = np.argsort(ids.ravel(), kind="stable")  # slots in (expert, slot) order
    np.testing.assert_array_equal(ids_sorted, order // topk)
    pos = np.empty_like(order)
    pos[order] = np.arange(order.size)
    np.testing.assert_array_equal(slotpos, pos)


def _brute_map(counts, offsets, bm, bn, n_cols, max_entries):
    out = []
    for ex, (c, off) in enumerate(zip(counts, offsets)):
        for mt in range((c + bm - 1) // bm):
            for nt in range(n_cols // bn):
                m0 = off + mt * bm
                out.append((m0, ex * n_cols + nt * bn, nt * bn, min(m0 + bm, off + c)))
    out += [(0, 0, 0, 0)] * (max_entries - len(out))
    return np.array(out[:max_entries], np.uint32)


@pytest.mark.parametrize("bm,gu_bn,dn_bn", [(128, 64, 64), (32, 64, 64), (128, 128, 256)])
def test_block_maps_brute_force(orc, rng, bm, gu_bn, dn_bn):
    m, e, topk, gu_n, dn_n = 1000, 64, 4, 1536, 2048
    ids = _routing(rng, m, e, topk)
    counts = orc.moe_count(ids, e)
    offsets = orc.moe_offsets(counts)
    gu_off, dn_off = orc.moe_block_offsets(counts, bm, gu_bn, dn_bn, gu_n, dn_n)
    m_tiles = -(-m * topk // bm) + e
    max_gu, max_dn = m_tiles * gu_n // gu_bn, m_tiles * dn_n // dn_bn
    gu, dn = orc.moe_blocks(counts, offsets, gu_off, dn_off, bm, gu_bn, dn_bn, gu_n, dn_n,
                            max_gu, max_dn)
    np.testing.assert_array_equal(gu, _brute_map(counts, offsets, bm, gu_bn, gu_n, max_gu))
    np.testing.assert_array_equal(dn, _brute_map(counts, offsets, bm, dn_bn, dn_n, max_dn))
    # every routed row appears in exactly one row tile of its expert, per column tile
    live = gu[gu[:, 0] < gu[:, 3]]
    cover = np.zeros(m * topk, int)
    for m0, _, n0, m_end in live:
        if n0 == 0:
            cover[m0:m_end] += 1
    assert (cover == 1).all()


def test_combine_closed_form(orc, rng):
    m, h, topk = 50, 64, 4
    sorted_rows = layout.synth_bf16(rng, (m * topk, h))
    slotpos = rng.permutation(m * topk).astype(np.uint32)
    w = layout.synth_bf16(rng, (m, topk), std=0.3)
    out = orc.moe_combine_rows(sorted_rows, slotpos, w, m, topk)
    acc = np.zeros((m, h), np.float32)
    for r in range(topk):
        prod = bf(w[:, r])[:, None] * bf(sorted_rows[slotpos.reshape(m, topk)[:, r]])
        acc = (acc + bf(layout.f32_to_bf16(prod.astype(np.float32)))).astype(np.float32)
    np.testing.assert_array_equal(out, layout.f32_to_bf16(acc))


def test_silu_mul_vs_float64(orc, rng):
    g = layout.synth_bf16(rng, (4096,), std=4.0)
    u = layout.synth_bf16(rng, (4096,), std=2.0)
    out = orc.silu_mul_bf16(g, u)
    gf = bf(g).astype(np.float64)
    ref = bf(layout.f32_to_bf16(gf / (1 + np.exp(-gf)))) * bf(u)
    np.testing.assert_allclose(bf(out), ref, rtol=2 ** -7, atol=1e-30)


def test_gather_rows(orc, rng):
    table = layout.synth_bf16(rng, (40, 32))
    ids = rng.integers(0, 40, 100).astype(np.uint32)
    np.testing.assert_array_equal(orc.gather_rows_bf16(table, ids), table[ids])


def test_grouped_gemm_is_per_expert_dense(orc, rng):
    e, n, k, bm, bn = 6, 128, 256, 32, 64
    w = layout.synth_quant(rng, e * n, k, 4)
    ids = rng.integers(0, e, (90, 1)).astype(np.uint32)
    counts = orc.moe_count(ids, e)
    offsets = orc.moe_offsets(counts)
    gu_off, dn_off = orc.moe_block_offsets(counts, bm, bn, bn, n, n)
    max_e = (-(-90 // bm) + e) * (n // bn)
    blocks, _ = orc.moe_blocks(counts, offsets, gu_off, dn_off, bm, bn, bn, n, n, max_e, max_e)
    a = layout.synth_bf16(rng, (90, k))
    c = orc.gemm_q4_grouped(a, w, blocks, max_e, n, bn)
    deq = bf(orc.dequant_bf16(w)).astype(np.float64)
    af = bf(a).astype(np.float64)
    for ex in range(e):
        rows = slice(offsets[ex], offsets[ex] + counts[ex])
        ref = af[rows] @ deq[ex * n:(ex + 1) * n].T
        got = bf(c[rows]).astype(np.float64)
        if counts[ex]:
            assert np.abs(got - ref).max() <= 2 ** -7 * np.abs(ref).max()


@pytest.mark.parametrize("mode", [0, 1])
def test_moe_prefill_composition_and_float64(orc, rng, mode):
    E, H, I, topk, m = 8, 256, 128, 2, 40
    gate, up, down = moe_weights(rng, E, H, I)
    router = router_weights(rng, E, H, f32=(mode == 0))
    bias = rng.normal(0, 0.05, E).astype(np.float32) if mode == 0 else None
    x = layout.synth_bf16(rng, (m, H))
    r = orc.moe_prefill(router, bias, mode, gate, up, down, E, topk, H, I, x)
    logits = orc.gemv_dense(router, x)
    ids, gw = orc.route(logits, bias, topk, mode)
    np.testing.assert_array_equal(r["ids"], ids)
    np.testing.assert_array_equal(r["gw"], gw)
    G, U, D = (bf(orc.dequant_bf16(q)).astype(np.float64) for q in (gate, up, down))
    xf = bf(x).astype(np.float64)
    out = np.zeros((m, H))
    for t in range(m):
        for j in range(topk):
            ex = ids[t, j]
            g = bf(layout.f32_to_bf16(G[ex * I:(ex + 1) * I] @ xf[t]))
            u = bf(layout.f32_to_bf16(U[ex * I:(ex + 1) * I] @ xf[t]))
            a = bf(layout.f32_to_bf16(bf(layout.f32_to_bf16(g / (1 + np.exp(-g.astype(np.float64))))) * u))
            p = D[ex * H:(ex + 1) * H] @ a.astype(np.float64)
            out[t] += bf(gw[t, j]) * p
    got = bf(r["out"]).astype(np.float64)
    assert np.linalg.norm(got - out) / np.linalg.norm(out) < 5e-3
    # masked run reproduces the selected tokens exactly and zeroes the rest
    mask = np.zeros(m, np.uint8)
    mask[[0, 7, 39]] = 1
    rm = orc.moe_prefill(router, bias, mode, gate, up, down, E, topk, H, I, x, token_mask=mask)
    np.testing.assert_array_equal(rm["out"][mask == 1], r["out"][mask == 1])
    assert not rm["out"][mask == 0].any()
