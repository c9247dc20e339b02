"""Pins the oracle's routing (a8, a12), decode expert GEMVs (a9-a11) and the
decode step composition (a19) against float64 and closed forms."""
import numpy as np
import pytest

from molten_amd import layout
from tests.synth import moe_weights

bf = layout.bf16_to_f32


def _rank(cand: np.ndarray, topk: int) -> list:
    """Greatest first, exact ties to the lower id (numpy lexsort)."""
    order = np.lexsort((np.arange(cand.size), -cand.astype(np.float64)))
    return order[:topk].tolist()


@pytest.mark.parametrize("mode", [0, 1])
def test_route_ranking_and_ties(orc, rng, mode):
    e, topk = 64, 4
    for trial in range(50):
        z = rng.normal(0, 2, e).astype(np.float32)
        if trial % 3 == 0:  # exact ties
            z[10] = z[20] = z[5] = np.float32(z.max() + 1.0)
        bias = rng.normal(0, 0.1, e).astype(np.float32) if mode == 0 else None
        ids, w = orc.route(z[None], bias, topk, mode)
        if mode == 0:
            s = np.array([1.0 / (1.0 + orc.expf(-float(v))) for v in z], np.float32)
            cand = (s + bias).astype(np.float32)
        else:
            cand = z
        assert ids[0].tolist() == _rank(cand, topk)
        if trial % 3 == 0 and mode == 1:
            assert ids[0][:3].tolist() == [5, 10, 20]


@pytest.mark.parametrize("mode", [0, 1])
def test_route_weights_closed_form(orc, rng, mode):
    e, topk = 64, 4
    z = rng.normal(0, 1, (200, e)).astype(np.float32)
    bias = rng.normal(0, 0.05, e).astype(np.float32)
    ids, w = orc.route(z, bias if mode == 0 else None, topk, mode, eps=1e-6)
    zz = z.astype(np.float64)
    chosen = np.take_along_axis(zz, ids.astype(np.int64), axis=1)
    if mode == 0:
        s = 1.0 / (1.0 + np.exp(-chosen))
        ref = s / (1e-6 + s.sum(axis=1, keepdims=True))
    else:
        ex = np.exp(chosen - chosen[:, :1])
        ref = ex / ex.sum(axis=1, keepdims=True)
        # softmax over all experts restricted to the chosen, renormalised
        full = np.exp(zz - zz.max(axis=1, keepdims=True))
        full = full / full.sum(axis=1, keepdims=True)
        sel = np.take_along_axis(full, ids.astype(np.int64), axis=1)
        np.testing.assert_allclose(sel / sel.sum(axis=1, keepdims=True), ref, rtol=1e-12)
    np.testing.assert_allclose(bf(w), ref, rtol=2 ** -8, atol=0)
    assert np.all(np.diff(bf(w), axis=1) <= 0) or mode == 0


def test_route_handles_all_equal_and_infinite(orc):
    z = np.zeros((1, 64), np.float32)
    ids, _ = orc.route(z, None, 4, 1)
    assert ids[0].tolist() == [0, 1, 2, 3]
    z = np.full((1, 8), -np.inf, np.float32)
    z[0, 6] = 1.0
    ids, _ = orc.route(z, None, 2, 1)
    assert ids[0].tolist() == [6, 0]


def test_gather_act_and_down_vs_float64(orc, rng):
    E, H, I, topk = 8, 512, 256, 4
    gate, up, down = moe_weights(rng, E, H, I)
    x = layout.synth_bf16(rng, (1, H))[0]
    ids = np.array([3, 0, 7, 5], np.uint32)
    act = orc.gather_act(gate, up, I, x, ids)
    xf = bf(x).astype(np.float64)
    G, U, D = gate.dequant_f64(), up.dequant_f64(), down.dequant_f64()
    for r, e in enumerate(ids):
        g = bf(layout.f32_to_bf16(G[e * I:(e + 1) * I] @ xf)).astype(np.float64)
        u = bf(layout.f32_to_bf16(U[e * I:(e + 1) * I] @ xf)).astype(np.float64)
        ref = bf(layout.f32_to_bf16(g / (1 + np.exp(-g)))).astype(np.float64) * u
        got = bf(act[r]).astype(np.float64)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 5e-3
    w = layout.f32_to_bf16(np.array([0.4, 0.3, 0.2, 0.1], np.float32))
    out = orc.down_combine(down, H, act, ids, w)
    ref = np.zeros(H)
    for r, e in enumerate(ids):
        p = D[e * H:(e + 1) * H] @ bf(act[r]).astype(np.float64)
        ref += bf(w[r]) * p
    got = bf(out).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 5e-3


def test_dense_gate_up_is_one_slot_gather(orc, rng):
    gate, up, _ = moe_weights(rng, 1, 256, 128)
    x = layout.synth_bf16(rng, (1, 256))[0]
    dense = orc.gather_act(gate, up, 128, x, None)
    routed = orc.gather_act(gate, up, 128, x, np.array([0], np.uint32))
    np.testing.assert_array_equal(dense, routed)


@pytest.mark.parametrize("mode,router_f32", [(0, True), (1, False)])
def test_moe_decode_is_the_composition(orc, rng, mode, router_f32):
    E, H, I, topk = 16, 512, 256, 4
    gate, up, down = moe_weights(rng, E, H, I)
    router = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    if not router_f32:
        router = layout.f32_to_bf16(router)
    bias = rng.normal(0, 0.05, E).astype(np.float32) if mode == 0 else None
    x = layout.synth_bf16(rng, (1, H))[0]
    r = orc.moe_decode(router, bias, mode, gate, up, down, E, topk, H, I, x)
    logits = orc.gemv_dense(router, x[None])
    np.testing.assert_array_equal(r["logits"], logits[0])
    ids, w = orc.route(logits, bias, topk, mode)
    np.testing.assert_array_equal(r["ids"], ids[0])
    np.testing.assert_array_equal(r["w"], w[0])
    act = orc.gather_act(gate, up, I, x, ids[0])
    np.testing.assert_array_equal(r["act"], act)
    np.testing.assert_array_equal(r["out"], orc.down_combine(down, H, act, ids[0], w[0]))
