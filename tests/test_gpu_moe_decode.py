"""GPU parity of the router, top-k and decode MoE expert kernels through the
C ABI.  Every output, float included, is compared bit
for bit: the kernels follow the oracle's chunk order and its exp."""
import numpy as np
import pytest

from molten_amd import hip, layout
from tests.devutil import dev_quant, empty_dev, from_dev, to_dev, zeros_dev
from tests.synth import moe_weights, router_weights

pytestmark = pytest.mark.gpu

E, H, I, TOPK = 64, 2048, 1536, 4


def _log(msg):
    print(msg, flush=True)


def _check_scratch(words, steps):
    """After `steps` single-launch decode steps each of the 256 workgroups'
    launch counts (words 0..255) equals steps, and word 256 (the three-launch
    path's done counter) is zero."""
    assert (words[:256] == steps).all(), words[:256]
    assert words[256] == 0


@pytest.fixture(scope="module")
def experts():
    """Config 3's 64 experts (uploaded once for the module)."""
    rng = np.random.default_rng(33)
    gate, up, down = moe_weights(rng, E, H, I)
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    dd, kd = dev_quant(down)
    return dict(h=(gate, up, down), d=(dg, du, dd), keep=(kg, ku, kd))


@pytest.mark.parametrize("f32", [True, False])
@pytest.mark.parametrize("n,k", [(64, 2048), (64, 4096), (100, 1536)])
def test_router_gemv_bit_exact(dev, orc, f32, n, k):
    rng = np.random.default_rng(n + k + f32)
    w = router_weights(rng, n, k, f32)
    x = layout.synth_bf16(rng, (1, k))
    y = empty_dev((n,), np.float32)
    (hip.gemv_f32 if f32 else hip.gemv_bf16)(to_dev(w), to_dev(x), y, n, k)
    np.testing.assert_array_equal(from_dev(y, np.float32).view(np.uint32),
                                  orc.gemv_dense(w, x)[0].view(np.uint32))


@pytest.mark.parametrize("mode", [0, 1])
def test_route_token_bit_exact(dev, orc, mode):
    rng = np.random.default_rng(4 + mode)
    for trial in range(20):
        z = rng.normal(0, 2, (1, E)).astype(np.float32)
        if trial % 4 == 0:
            z[0, 7] = z[0, 40] = np.float32(z.max() + 0.5)
        bias = rng.normal(0, 0.1, E).astype(np.float32) if mode == 0 else None
        ids = empty_dev((TOPK,), np.uint32)
        w = empty_dev((TOPK,), np.uint16)
        hip.route_token(to_dev(z), None if bias is None else to_dev(bias), ids, w, E, TOPK, mode)
        want_ids, want_w = orc.route(z, bias, TOPK, mode)
        assert from_dev(ids, np.uint32).tolist() == want_ids[0].tolist()
        np.testing.assert_array_equal(from_dev(w, np.uint16), want_w[0])


@pytest.mark.parametrize("mode,f32", [(0, True), (1, False)])
def test_router_route_fused(dev, orc, mode, f32):
    rng = np.random.default_rng(9 + mode)
    w = router_weights(rng, E, H, f32)
    bias = rng.normal(0, 0.05, E).astype(np.float32) if mode == 0 else None
    wd = to_dev(w)
    bd = None if bias is None else to_dev(bias)
    counter = zeros_dev((1,), np.uint32)
    logits = empty_dev((E,), np.float32)
    ids = empty_dev((TOPK,), np.uint32)
    wt = empty_dev((TOPK,), np.uint16)
    for trial in range(8):
        x = layout.synth_bf16(rng, (1, H))
        hip.router_route(wd, to_dev(x), logits, bd, ids, wt, counter, E, H, TOPK, mode)
        want_logits = orc.gemv_dense(w, x)
        want_ids, want_w = orc.route(want_logits, bias, TOPK, mode)
        np.testing.assert_array_equal(from_dev(logits, np.float32), want_logits[0])
        assert from_dev(ids, np.uint32).tolist() == want_ids[0].tolist()
        np.testing.assert_array_equal(from_dev(wt, np.uint16), want_w[0])
        assert from_dev(counter, np.uint32)[0] == 0


def test_gather_act_bit_exact(dev, orc, experts):
    gate, up, down = experts["h"]
    dg, du, dd = experts["d"]
    rng = np.random.default_rng(1)
    for trial in range(3):
        x = layout.synth_bf16(rng, (1, H))[0]
        ids = rng.choice(E, TOPK, replace=False).astype(np.uint32)
        act = empty_dev((TOPK, I), np.uint16)
        hip.gemv_gather_act(dg, du, to_dev(x), to_dev(ids), act, TOPK, I)
        np.testing.assert_array_equal(from_dev(act, np.uint16), orc.gather_act(gate, up, I, x, ids))


def test_gu_act_dense_bit_exact(dev, orc):
    rng = np.random.default_rng(3)
    n, k = 11776, 2048  # the model's dense FFN
    gate = layout.synth_quant(rng, n, k, 4)
    up = layout.synth_quant(rng, n, k, 4)
    x = layout.synth_bf16(rng, (1, k))[0]
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    act = empty_dev((n,), np.uint16)
    hip.gemv_gu_act(dg, du, to_dev(x), act)
    np.testing.assert_array_equal(from_dev(act, np.uint16), orc.gather_act(gate, up, n, x, None)[0])


@pytest.mark.parametrize("topk", [4, 2, 1])
def test_down_combine_bit_exact(dev, orc, experts, topk):
    gate, up, down = experts["h"]
    dg, du, dd = experts["d"]
    rng = np.random.default_rng(10 + topk)
    act = layout.synth_bf16(rng, (topk, I), std=2.0)
    ids = rng.choice(E, topk, replace=False).astype(np.uint32)
    w = layout.f32_to_bf16(rng.dirichlet(np.ones(topk)).astype(np.float32))
    out = empty_dev((H,), np.uint16)
    hip.gemv_gather_down_combine4(dd, to_dev(act), to_dev(ids), to_dev(w), out, topk, H)
    np.testing.assert_array_equal(from_dev(out, np.uint16), orc.down_combine(down, H, act, ids, w))


@pytest.mark.parametrize("huge", [False, True])
def test_expert_kernels_extreme_activations(dev, orc, experts, huge):
    """gather_act and down_combine with denormal / signed-zero / 2^100-scale
    inputs (the latter forces the convert form of the Q4 dot)."""
    gate, up, down = experts["h"]
    dg, du, dd = experts["d"]
    rng = np.random.default_rng(20 + huge)

    def extreme(shape, scale):
        v = rng.normal(0, 1, shape).astype(np.float32)
        flat = v.reshape(-1)
        idx = rng.choice(flat.size, 48, replace=False)
        flat[idx[:16]] = np.float32(2.0 ** -130)
        flat[idx[16:24]] = -0.0
        if huge:
            flat[idx[24:28]] = np.float32(scale)
        return layout.f32_to_bf16(v)

    x = extreme((H,), 2.0 ** 106)
    ids = rng.choice(E, TOPK, replace=False).astype(np.uint32)
    act = empty_dev((TOPK, I), np.uint16)
    hip.gemv_gather_act(dg, du, to_dev(x), to_dev(ids), act, TOPK, I)
    np.testing.assert_array_equal(from_dev(act, np.uint16), orc.gather_act(gate, up, I, x, ids))
    a = extreme((TOPK, I), 2.0 ** 105)
    w = layout.f32_to_bf16(np.full(TOPK, 0.25, np.float32))
    out = empty_dev((H,), np.uint16)
    hip.gemv_gather_down_combine4(dd, to_dev(a), to_dev(ids), to_dev(w), out, TOPK, H)
    want = orc.down_combine(down, H, a, ids, w)
    assert np.isfinite(layout.bf16_to_f32(want)).all()
    np.testing.assert_array_equal(from_dev(out, np.uint16), want)


@pytest.mark.parametrize("mode,f32", [(1, False), (0, True)])
def test_moe_decode_step_bit_exact(dev, orc, experts, mode, f32):
    """Config 3: router -> top-4 -> gate/up/SwiGLU -> down -> combine, all
    intermediates and the output bit-exact, for several inputs (different
    routings), with the scratch words consistent between steps."""
    _log(f"moe decode mode={mode} f32={f32}")
    gate, up, down = experts["h"]
    dg, du, dd = experts["d"]
    rng = np.random.default_rng(100 + mode)
    router = router_weights(rng, E, H, f32)
    bias = rng.normal(0, 0.05, E).astype(np.float32) if mode == 0 else None
    rd = to_dev(router)
    bd = None if bias is None else to_dev(bias)
    out = empty_dev((H,), np.uint16)
    logits = empty_dev((E,), np.float32)
    ids = empty_dev((TOPK,), np.uint32)
    wt = empty_dev((TOPK,), np.uint16)
    act = empty_dev((TOPK, I), np.uint16)
    scratch = zeros_dev((hip.MOE_DECODE_SCRATCH_WORDS,), np.uint32)
    seen = set()
    for trial in range(4):
        x = layout.synth_bf16(rng, (1, H))[0]
        hip.moe_decode(rd, bd, dg, du, dd, E, TOPK, to_dev(x), out, logits, ids, wt, act, scratch,
                       mode=mode)
        want = orc.moe_decode(router, bias, mode, gate, up, down, E, TOPK, H, I, x)
        assert from_dev(ids, np.uint32).tolist() == want["ids"].tolist()
        np.testing.assert_array_equal(from_dev(logits, np.float32), want["logits"])
        np.testing.assert_array_equal(from_dev(wt, np.uint16), want["w"])
        np.testing.assert_array_equal(from_dev(act, np.uint16), want["act"])
        np.testing.assert_array_equal(from_dev(out, np.uint16), want["out"])
        _check_scratch(from_dev(scratch, np.uint32), trial + 1)
        seen.add(tuple(want["ids"].tolist()))
    assert len(seen) > 1  # the inputs exercised different routings


@pytest.mark.parametrize("e,h,i,topk,shifted", [(8, 512, 256, 2, False), (16, 1024, 128, 1, False),
                                                 (32, 768, 192, 3, False), (8, 512, 128, 2, True)])
def test_moe_decode_step_shapes(dev, orc, e, h, i, topk, shifted):
    """Decode step at other shapes and top-k, bit-exact, over repeated steps
    sharing one scratch.  Activations that are not 4-byte aligned (shifted)
    take the three-launch path instead of the single-launch kernel."""
    _log(f"moe decode shape e={e} h={h} i={i} topk={topk} shifted={shifted}")
    rng = np.random.default_rng(7 * e + i + topk)
    gate, up, down = moe_weights(rng, e, h, i)
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    dd, kd = dev_quant(down)
    router = router_weights(rng, e, h, False)
    rd = to_dev(router)
    out = empty_dev((h,), np.uint16)
    logits = empty_dev((e,), np.float32)
    ids = empty_dev((topk,), np.uint32)
    wt = empty_dev((topk,), np.uint16)
    act = empty_dev((topk * i + 1,), np.uint16)[1:] if shifted else empty_dev((topk * i,), np.uint16)
    assert (act.data_ptr() % 4 != 0) == shifted
    scratch = zeros_dev((hip.MOE_DECODE_SCRATCH_WORDS,), np.uint32)
    for trial in range(3):
        x = layout.synth_bf16(rng, (1, h))[0]
        hip.moe_decode(rd, None, dg, du, dd, e, topk, to_dev(x), out, logits, ids, wt, act, scratch,
                       mode=1)
        want = orc.moe_decode(router, None, 1, gate, up, down, e, topk, h, i, x)
        assert from_dev(ids, np.uint32).tolist() == want["ids"].tolist()
        np.testing.assert_array_equal(from_dev(logits, np.float32), want["logits"])
        np.testing.assert_array_equal(from_dev(wt, np.uint16), want["w"])
        np.testing.assert_array_equal(from_dev(act, np.uint16).reshape(topk, i), want["act"])
        np.testing.assert_array_equal(from_dev(out, np.uint16), want["out"])
        _check_scratch(from_dev(scratch, np.uint32), 0 if shifted else trial + 1)
    del kg, ku, kd


def test_moe_decode_wide_intermediate_is_rejected(dev, orc):
    """An intermediate size above 2048 (a slot's down chunks no longer fit one
    butterfly's 64 lanes, and the three-launch path holds act in registers)
    is refused with MH_ERR_UNSUPPORTED instead of a partial down dot."""
    _log("moe decode e=4 h=512 i=4096 topk=2 (rejected)")
    e, h, i, topk = 4, 512, 4096, 2
    rng = np.random.default_rng(4096)
    gate, up, down = moe_weights(rng, e, h, i)
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    dd, kd = dev_quant(down)
    rd = to_dev(router_weights(rng, e, h, False))
    out = empty_dev((h,), np.uint16)
    logits = empty_dev((e,), np.float32)
    ids = empty_dev((topk,), np.uint32)
    wt = empty_dev((topk,), np.uint16)
    act = empty_dev((topk * i,), np.uint16)
    scratch = zeros_dev((hip.MOE_DECODE_SCRATCH_WORDS,), np.uint32)
    x = layout.synth_bf16(rng, (1, h))[0]
    with pytest.raises(hip.MoltenError) as ei:
        hip.moe_decode(rd, None, dg, du, dd, e, topk, to_dev(x), out, logits, ids, wt, act, scratch,
                       mode=1)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    import torch

    torch.cuda.synchronize()
    del kg, ku, kd


def test_prefill_router_and_route_batch(dev, orc):
    rng = np.random.default_rng(77)
    m = 300
    w = router_weights(rng, E, H, False)
    x = layout.synth_bf16(rng, (m, H))
    logits = empty_dev((m, E), np.float32)
    hip.router_prefill(to_dev(x), to_dev(w), logits, m, H, E)
    want = orc.gemv_dense(w, x)
    np.testing.assert_array_equal(from_dev(logits, np.float32), want)
    ids = empty_dev((m, TOPK), np.uint32)
    gw = empty_dev((m, TOPK), np.uint16)
    hip.moe_route_batch(logits, None, ids, gw, m, E, TOPK, mode=1)
    want_ids, want_w = orc.route(want, None, TOPK, 1)
    np.testing.assert_array_equal(from_dev(ids, np.uint32), want_ids)
    np.testing.assert_array_equal(from_dev(gw, np.uint16), want_w)


@pytest.mark.parametrize("e", [64, 100, 256])
def test_route_special_values_match_serial_scan(dev, orc, e):
    """NaN and -inf candidates never win, exact ties go to the lower id, and a
    token with fewer eligible experts than slots falls back to expert 0, as
    the serial scan of the reference does."""
    rng = np.random.default_rng(e)
    topk = 4
    cases = []
    z = rng.normal(0, 1, e).astype(np.float32)
    z[[3, 9]] = np.nan
    z[[5, 6]] = -np.inf
    cases.append(z)
    z = np.full(e, -np.inf, np.float32)
    z[e - 1] = 2.0
    z[7] = 2.0
    cases.append(z)                       # two eligible, both tied
    cases.append(np.full(e, np.nan, np.float32))  # none eligible
    z = np.zeros(e, np.float32)
    z[e // 2] = np.inf
    cases.append(z)
    m = len(cases)
    logits = np.stack(cases)
    for mode in (0, 1):
        bias = rng.normal(0, 0.1, e).astype(np.float32) if mode == 0 else None
        ids = empty_dev((m, topk), np.uint32)
        w = empty_dev((m, topk), np.uint16)
        hip.moe_route_batch(to_dev(logits), None if bias is None else to_dev(bias), ids, w, m, e,
                            topk, mode=mode)
        want_ids, want_w = orc.route(logits, bias, topk, mode)
        np.testing.assert_array_equal(from_dev(ids, np.uint32), want_ids)
        np.testing.assert_array_equal(from_dev(w, np.uint16), want_w)


def test_moe_decode_expired_wait_is_reported(dev, orc):
    """The single-launch decode step's bounded waits give up when one
    workgroup's launch count (planted from the host) is ahead of the others':
    its logits and activations carry an epoch no other workgroup waits for,
    so every wait runs to its bound and the kernel still ends normally.  The
    output is NaN and MH_STATUS_DECODE_WAIT is set; after the caller re-zeroes
    the scratch the next step is bit-exact again."""
    e, h, i, topk = 8, 512, 256, 2
    _log(f"moe decode expired wait e={e} h={h} i={i} topk={topk}")
    rng = np.random.default_rng(808)
    gate, up, down = moe_weights(rng, e, h, i)
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    dd, kd = dev_quant(down)
    router = router_weights(rng, e, h, False)
    rd = to_dev(router)
    x = layout.synth_bf16(rng, (1, h))[0]
    out = empty_dev((h,), np.uint16)
    logits = empty_dev((e,), np.float32)
    ids = empty_dev((topk,), np.uint32)
    wt = empty_dev((topk,), np.uint16)
    act = empty_dev((topk, i), np.uint16)
    words = np.zeros(hip.MOE_DECODE_SCRATCH_WORDS, np.uint32)
    words[5] = 100  # workgroup 5's launch count
    scratch = to_dev(words)
    hip.device_status(clear=True)
    hip.moe_decode(rd, None, dg, du, dd, e, topk, to_dev(x), out, logits, ids, wt, act, scratch, mode=1)
    got = from_dev(out, np.uint16)
    assert (got == 0x7FC0).all(), got[:8]
    assert hip.device_status(clear=True) & hip.STATUS_DECODE_WAIT
    scratch.zero_()
    hip.moe_decode(rd, None, dg, du, dd, e, topk, to_dev(x), out, logits, ids, wt, act, scratch, mode=1)
    want = orc.moe_decode(router, None, 1, gate, up, down, e, topk, h, i, x)
    np.testing.assert_array_equal(from_dev(out, np.uint16), want["out"])
    assert hip.device_status(clear=True) == 0
    del kg, ku, kd


def _prefix_experts(h, n_exp, rows_per_expert):
    """The first n_exp experts of stacked HostQuant h (a view of its rows)."""
    n = n_exp * rows_per_expert
    return layout.HostQuant(h.codes[:n], h.scales[:n], h.biases[:n], n, h.k, h.group_size, h.bits)


@pytest.mark.parametrize("n_exp,mode", [(32, 1), (48, 0), (5, 1)])
def test_moe_decode_config3_shape_fewer_experts(dev, orc, experts, n_exp, mode):
    """d_model 2048, intermediate 1536, top-4 over fewer than 64 experts
    (the single launch with router workgroups past E idle), both routing
    modes, bit-exact over repeated steps."""
    _log(f"moe decode config-3 shape with {n_exp} experts mode={mode}")
    gate, up, down = (_prefix_experts(experts["h"][0], n_exp, I), _prefix_experts(experts["h"][1], n_exp, I),
                      _prefix_experts(experts["h"][2], n_exp, H))
    dg, kg = dev_quant(gate)
    du, ku = dev_quant(up)
    dd, kd = dev_quant(down)
    rng = np.random.default_rng(900 + n_exp)
    router = router_weights(rng, n_exp, H, False)
    bias = rng.normal(0, 0.05, n_exp).astype(np.float32) if mode == 0 else None
    rd = to_dev(router)
    bd = None if bias is None else to_dev(bias)
    out = empty_dev((H,), np.uint16)
    logits = empty_dev((n_exp,), np.float32)
    ids = empty_dev((TOPK,), np.uint32)
    wt = empty_dev((TOPK,), np.uint16)
    act = empty_dev((TOPK, I), np.uint16)
    scratch = zeros_dev((hip.MOE_DECODE_SCRATCH_WORDS,), np.uint32)
    for trial in range(3):
        x = layout.synth_bf16(rng, (1, H))[0]
        hip.moe_decode(rd, bd, dg, du, dd, n_exp, TOPK, to_dev(x), out, logits, ids, wt, act, scratch, mode=mode)
        want = orc.moe_decode(router, bias, mode, gate, up, down, n_exp, TOPK, H, I, x)
        assert from_dev(ids, np.uint32).tolist() == want["ids"].tolist()
        np.testing.assert_array_equal(from_dev(logits, np.float32), want["logits"])
        np.testing.assert_array_equal(from_dev(wt, np.uint16), want["w"])
        np.testing.assert_array_equal(from_dev(act, np.uint16), want["act"])
        np.testing.assert_array_equal(from_dev(out, np.uint16), want["out"])
        _check_scratch(from_dev(scratch, np.uint32), trial + 1)
    del kg, ku, kd


def test_moe_decode_alternating_shapes_share_scratch(dev, orc, experts):
    """Single-launch steps at config 3's shape and at a small shape alternate
    on one scratch buffer: the launch counts stay in lockstep and every step
    is bit-exact."""
    _log("moe decode alternating shapes on one scratch")
    gate, up, down = experts["h"]
    dg, du, dd = experts["d"]
    rng = np.random.default_rng(4242)
    router = router_weights(rng, E, H, False)
    rd = to_dev(router)
    e2, h2, i2, k2 = 8, 512, 256, 2
    g2, u2, d2 = moe_weights(rng, e2, h2, i2)
    dg2, kg = dev_quant(g2)
    du2, ku = dev_quant(u2)
    dd2, kd = dev_quant(d2)
    router2 = router_weights(rng, e2, h2, False)
    rd2 = to_dev(router2)
    scratch = zeros_dev((hip.MOE_DECODE_SCRATCH_WORDS,), np.uint32)
    for trial in range(4):
        if trial % 2 == 0:
            x = layout.synth_bf16(rng, (1, H))[0]
            out, logits = empty_dev((H,), np.uint16), empty_dev((E,), np.float32)
            ids, wt, act = empty_dev((TOPK,), np.uint32), empty_dev((TOPK,), np.uint16), empty_dev((TOPK, I), np.uint16)
            hip.moe_decode(rd, None, dg, du, dd, E, TOPK, to_dev(x), out, logits, ids, wt, act, scratch, mode=1)
            want = orc.moe_decode(router, None, 1, gate, up, down, E, TOPK, H, I, x)
        else:
            x = layout.synth_bf16(rng, (1, h2))[0]
            out, logits = empty_dev((h2,), np.uint16), empty_dev((e2,), np.float32)
            ids, wt, act = empty_dev((k2,), np.uint32), empty_dev((k2,), np.uint16), empty_dev((k2, i2), np.uint16)
            hip.moe_decode(rd2, None, dg2, du2, dd2, e2, k2, to_dev(x), out, logits, ids, wt, act, scratch, mode=1)
            want = orc.moe_decode(router2, None, 1, g2, u2, d2, e2, k2, h2, i2, x)
        assert from_dev(ids, np.uint32).tolist() == want["ids"].tolist()
        np.testing.assert_array_equal(from_dev(act, np.uint16).reshape(want["act"].shape), want["act"])
        np.testing.assert_array_equal(from_dev(out, np.uint16), want["out"])
        _check_scratch(from_dev(scratch, np.uint32), trial + 1)
    del kg, ku, kd


def test_moe_decode_config3_expired_wait_is_reported(dev, orc, experts):
    """The single-launch decode step at config 3's shape with workgroup 5's
    launch count planted ahead from the host: its router row and
    activations carry an epoch no other workgroup waits for, so the bounded
    waits give up and the kernel ends normally.  Every output is NaN and
    MH_STATUS_DECODE_WAIT is set; after the caller re-zeroes the scratch the
    next step is bit-exact again."""
    _log("moe decode config-3 shape, planted launch count")
    gate, up, down = experts["h"]
    dg, du, dd = experts["d"]
    rng = np.random.default_rng(809)
    router = router_weights(rng, E, H, False)
    rd = to_dev(router)
    x = layout.synth_bf16(rng, (1, H))[0]
    out = empty_dev((H,), np.uint16)
    logits = empty_dev((E,), np.float32)
    ids = empty_dev((TOPK,), np.uint32)
    wt = empty_dev((TOPK,), np.uint16)
    act = empty_dev((TOPK, I), np.uint16)
    words = np.zeros(hip.MOE_DECODE_SCRATCH_WORDS, np.uint32)
    words[5] = 100
    scratch = to_dev(words)
    hip.device_status(clear=True)
    hip.moe_decode(rd, None, dg, du, dd, E, TOPK, to_dev(x), out, logits, ids, wt, act, scratch, mode=1)
    got = from_dev(out, np.uint16)
    assert (got == 0x7FC0).all(), got[:8]
    assert hip.device_status(clear=True) & hip.STATUS_DECODE_WAIT
    scratch.zero_()
    hip.moe_decode(rd, None, dg, du, dd, E, TOPK, to_dev(x), out, logits, ids, wt, act, scratch, mode=1)
    want = orc.moe_decode(router, None, 1, gate, up, down, E, TOPK, H, I, x)
    np.testing.assert_array_equal(from_dev(out, np.uint16), want["out"])
    assert hip.device_status(clear=True) == 0
