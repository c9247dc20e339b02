#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul hot path.

One step = one pass of the hot path over one batch of synthetic input with
all inputs resident in HBM.  The headline line is BASELINE config 2 (the Q4
LM head 65536 x 2048 GEMV with fused argmax: logits stored and the token id
written by the same launch), in GB/s of algorithmic bytes.  The other
BASELINE configs are measured in the same run and reported under "others":

  config 1  Q4 GEMV 2048 x 2048, batch 1                 GB/s (HBM)
  config 3  MoE decode step (router, top-4 of 64, experts) GB/s (HBM)
  config 4  prefill MoE, 4096 tokens x top-4 of 64        TFLOP/s (bf16 MFMA)
  config 5  Q6 LM head 65536 x 2048 + argmax, b=1 / b=8   GB/s (HBM)

Weights are synthetic (BASELINE distributions, random-init, generated on the
GPU) and rotated over enough copies (>= 300 MB) that the 256 MB Infinity
Cache cannot hold the working set; the MoE inputs vary per step so routing
changes.  The timed steps are captured in one HIP graph and replayed between
HIP events on the launch stream (no host launch overhead in the timing).
The CPU baseline is the C oracle timed on the host cores on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA

# Algorithmic bytes per step: every weight byte (codes, scales, biases) read
# once, plus the inputs and outputs.
BYTES = {
    "config1": 2_367_488,
    "config2": 75_632_644,
    "config3": 21_504_000,
    "config5_b1": 109_187_076,
    "config5_b8": 110_133_280,
    # the decode epilogue variants (proj3, conv3) at the model's shapes
    "next_proj3_gemv_scatter": 3_549_184,  # 3072 rows x (1024 code + 128 s/b) B + x + outputs
    "next_conv3_gemv": 7_114_752,          # 6144 rows x 1152 B + x + taps + state in/out + out
    "next_dense_down_q4_k11776": 13_593_600,  # 2048 rows x (5888 code + 736 s/b) B + x + y
    "next_gather_rows_q6_4096": 23_609_344,   # 4096 x (1536 code + 128 s/b + 4096 out) B + ids
    "next_sample_gumbel_128000": 272_008,  # 128000 bf16 logits + the seen bits + the key
    # logits + seen read, w written once and read by 6 radix rounds and the draw
    "next_sample_topk_topp_128000": 272_008 + 128_000 * 4 * 8,
    "next_token_tail_embed": 13_972,  # key read + clear, token, one Q6 row + s/b, gain, x and normed rows
}
FLOPS_CONFIG4 = 309_237_645_312


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_quant(torch, n, k, bits, copies, dev, gen):
    from molten_amd import hip

    out = []
    for _ in range(copies):
        words = k * bits // 32
        codes = torch.randint(-2**31, 2**31 - 1, (n, words), dtype=torch.int32, device=dev,
                              generator=gen)
        g = k // 64
        scales = (torch.randn(n, g, device=dev, generator=gen).abs() * 0.02 + 1e-3)
        biases = torch.randn(n, g, device=dev, generator=gen) * 0.02
        scales = scales.to(torch.bfloat16).view(torch.int16)
        biases = biases.to(torch.bfloat16).view(torch.int16)
        out.append((hip.QuantWeights(codes, scales, biases, n, k, 64, bits), (codes, scales, biases)))
    return out


def bf16_randn(torch, shape, dev, gen, std=1.0):
    return (torch.randn(shape, device=dev, generator=gen) * std).to(torch.bfloat16).view(torch.int16)


EAGER = False  # --eager: no graph capture (counter collection sees only eager dispatches)


def timed(torch, fn, steps, warmup):
    """Average ms per call of fn(i) over `steps` calls after `warmup` eager
    calls.  The `steps` calls are captured once in a HIP graph; the graph is
    replayed five times, each replay between two events on the launch stream
    and bracketed by synchronizes, and the median replay is returned.  Host
    launch overhead (ctypes, Python) is not timed: the GPU runs the kernels
    back to back, as a decode loop captured in a graph would.  With EAGER the
    `steps` calls are launched directly between the two events instead."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    if EAGER:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            fn(warmup + i)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            fn(warmup + i)
    graph.replay()  # untimed first replay
    torch.cuda.synchronize()
    times = []
    for _ in range(5):  # median of five timed replays
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    del graph
    return sorted(times)[len(times) // 2]


def bench_lm_head(torch, hip, dev, gen, bits, batch, steps, warmup, copies):
    n, k = 65536, 2048
    ws = make_quant(torch, n, k, bits, copies, dev, gen)
    x = bf16_randn(torch, (batch, k), dev, gen)
    y = torch.empty((batch, n), dtype=torch.int16, device=dev)
    scratch = torch.zeros(hip.argmax_scratch_words(batch), dtype=torch.int64, device=dev)
    ids = torch.empty(batch, dtype=torch.int32, device=dev)

    def step(i):
        hip.gemv_quant_argmax(ws[i % copies][0], x, y, scratch, ids, batch)

    ms = timed(torch, step, steps, warmup)
    del ws
    return ms


def bench_config1(torch, hip, dev, gen, steps, warmup):
    copies = 128  # 128 x 2.36 MB = 302 MB
    ws = make_quant(torch, 2048, 2048, 4, copies, dev, gen)
    x = bf16_randn(torch, (1, 2048), dev, gen)
    y = torch.empty((1, 2048), dtype=torch.int16, device=dev)
    ms = timed(torch, lambda i: hip.gemv_quant(ws[i % copies][0], x, y, 1), steps, warmup)
    del ws
    return ms


def bench_next_rows(torch, hip, dev, gen, steps, warmup):
    """The decode epilogue variants at the model's shapes: proj3 (Q 2048, K 512,
    V 512 rows into a 4096-position cache) and conv3 (H 2048)."""
    copies = 96  # 96 x 3.5 MB and 48 x 7.1 MB: beyond the 256 MB Infinity Cache
    qs = make_quant(torch, 2048, 2048, 4, copies, dev, gen)
    ks = make_quant(torch, 512, 2048, 4, copies, dev, gen)
    vs = make_quant(torch, 512, 2048, 4, copies, dev, gen)
    x = bf16_randn(torch, (2048,), dev, gen)
    q = torch.empty(2048, dtype=torch.int16, device=dev)
    k = torch.empty(512, dtype=torch.int16, device=dev)
    cache = torch.empty((8, 4096, 64), dtype=torch.int16, device=dev)
    ms_p = timed(torch, lambda i: hip.proj3_gemv_scatter(qs[i % copies][0], ks[i % copies][0], vs[i % copies][0],
                                                         x, q, k, cache, 4096, i % 4096), steps, warmup)
    del qs, ks, vs
    H = 2048
    ws = make_quant(torch, 3 * H, 2048, 4, copies // 2, dev, gen)
    taps = bf16_randn(torch, (H, 3), dev, gen, std=0.5)
    states = [bf16_randn(torch, (2, H), dev, gen) for _ in range(2)]
    out = torch.empty(H, dtype=torch.int16, device=dev)
    ms_c = timed(torch, lambda i: hip.conv3_gemv(ws[i % (copies // 2)][0], x, taps, states[i % 2], out,
                                                 states[(i + 1) % 2]), steps, warmup)
    del ws
    # the dense FFN down projection (lfm_gemv_q4_bf16_k11776): 2048 x 11776
    ds = make_quant(torch, 2048, 11776, 4, 24, dev, gen)  # 24 x 13.6 MB
    xd = bf16_randn(torch, (1, 11776), dev, gen)
    yd = torch.empty((1, 2048), dtype=torch.int16, device=dev)
    ms_d = timed(torch, lambda i: hip.gemv_quant(ds[i % 24][0], xd, yd, 1), steps, warmup)
    del ds
    # the Q6 embedding table (65536 x 2048): prefill gather of 4096 rows and
    # the decode token tail (key -> token, its row + RMSNorm)
    tab = make_quant(torch, 65536, 2048, 6, 1, dev, gen)[0]
    ids = [torch.randint(0, 65536, (4096,), dtype=torch.int32, device=dev, generator=gen) for _ in range(4)]
    gout = torch.empty((4096, 2048), dtype=torch.int16, device=dev)
    ms_g = timed(torch, lambda i: hip.gather_rows_q6(tab[0], ids[i % 4], 4096, gout), steps, warmup)
    keys = torch.randint(0, 65536, (steps + warmup + 8,), dtype=torch.int64, device=dev, generator=gen)
    keys = (keys ^ 0xffffffff) | (0x40000000 << 32)  # low word ~token
    best = torch.empty(1, dtype=torch.int64, device=dev)
    tok = torch.empty(1, dtype=torch.int32, device=dev)
    gain = bf16_randn(torch, (2048,), dev, gen)
    xe = torch.empty(2048, dtype=torch.int16, device=dev)
    ne = torch.empty(2048, dtype=torch.int16, device=dev)

    def tail(i):  # (timed with the copy that refills the key the tail clears)
        best.copy_(keys[i:i + 1])
        hip.token_tail_embed(best, tok, tab[0], gain, xe, ne, 1e-5)

    ms_t = timed(torch, tail, steps, warmup)
    del tab
    # the temperature-only Gumbel draw over a stored 128000-logit row
    from molten_amd.hip import sample_params
    rows = [bf16_randn(torch, (128000,), dev, gen, std=3.0) for _ in range(4)]
    seen = torch.randint(-2**31, 2**31 - 1, (4000,), dtype=torch.int32, device=dev, generator=gen)
    key = torch.zeros(1, dtype=torch.int64, device=dev)
    prm = [sample_params(0.8, 1234, i, 1.1) for i in range(8)]
    ms_s = timed(torch, lambda i: hip.sample_gumbel(rows[i % 4], 128000, seen, prm[i % 8], key), steps, warmup)
    # the kept-set draw (top_k 40 then top_p 0.9) on the same rows
    wsb = hip.sample_workspace_bytes(128000)
    sws = torch.zeros(wsb, dtype=torch.uint8, device=dev)
    prm_kp = [sample_params(0.8, 1234, i, 1.1, top_k=40, top_p=0.9) for i in range(8)]
    ms_kp = timed(torch, lambda i: hip.sample_draw(rows[i % 4], 128000, seen, prm_kp[i % 8], key, sws, wsb),
                  steps, warmup)
    # the prefill dense projections (dequant + GEMM fused), 4096 tokens: an
    # attention projection 2048 -> 2048 and the dense FFN gate 2048 -> 11776
    ms_x = []
    pa = bf16_randn(torch, (4096, 2048), dev, gen)
    for n in (2048, 11776):
        pw = make_quant(torch, n, 2048, 4, 4, dev, gen)
        pc = torch.empty((4096, n), dtype=torch.int16, device=dev)
        ms_x.append(timed(torch, lambda i: hip.gemm_q4_dense(pa, 4096, pw[i % 4][0], pc), steps, warmup))
        del pw, pc
    # the unfused pair the reference's project() runs for weights the fused
    # path does not take: a dense bf16 GEMM over an already dequantized W,
    # and the generic quantized GEMM (dequantize into scratch + that GEMM)
    pb = [bf16_randn(torch, (2048, 2048), dev, gen, std=0.05) for _ in range(4)]
    pc = torch.empty((4096, 2048), dtype=torch.int16, device=dev)
    ms_x.append(timed(torch, lambda i: hip.gemm_bf16_nt(pa, pb[i % 4], pc, 4096, 2048, 2048), steps, warmup))
    pw = make_quant(torch, 2048, 2048, 4, 4, dev, gen)
    scr = torch.empty(2048 * 2048, dtype=torch.int16, device=dev)
    ms_x.append(timed(torch, lambda i: hip.gemm_quant_bf16_nt(pa, 4096, pw[i % 4][0], pc, scr, 2048 * 2048),
                      steps, warmup))
    del pb, pc, pw, scr
    return ms_p, ms_c, ms_d, ms_g, ms_t, ms_x, (ms_s, ms_kp)


def moe_set(torch, dev, gen, E=64, H=2048, I=1536):
    gate = make_quant(torch, E * I, H, 4, 1, dev, gen)[0]
    up = make_quant(torch, E * I, H, 4, 1, dev, gen)[0]
    down = make_quant(torch, E * H, I, 4, 1, dev, gen)[0]
    router = bf16_randn(torch, (E, H), dev, gen, std=0.02)
    return gate, up, down, router


def bench_config3(torch, hip, dev, gen, steps, warmup):
    E, H, I, topk = 64, 2048, 1536, 4
    sets = [moe_set(torch, dev, gen) for _ in range(4)]  # 4 x 340 MB of experts
    xs = [bf16_randn(torch, (H,), dev, gen) for _ in range(16)]
    out = torch.empty(H, dtype=torch.int16, device=dev)
    logits = torch.empty(E, dtype=torch.float32, device=dev)
    ids = torch.empty(topk, dtype=torch.int32, device=dev)
    wt = torch.empty(topk, dtype=torch.int16, device=dev)
    act = torch.empty((topk, I), dtype=torch.int16, device=dev)
    scratch = torch.zeros(hip.MOE_DECODE_SCRATCH_WORDS, dtype=torch.int32, device=dev)

    def step(i):
        g, u, d, r = sets[i % len(sets)]
        hip.moe_decode(r, None, g[0], u[0], d[0], E, topk, xs[i % len(xs)], out, logits, ids, wt,
                       act, scratch, mode=hip.ROUTE_SOFTMAX)

    ms = timed(torch, step, steps, warmup)
    del sets
    return ms


TIMELINE_PHASES = ("start", "logit_stored", "routed", "gate_up_issued", "first_act_published",
                   "last_act_published", "down_issued", "acts_exchanged", "out_stored")


def timeline_config3(torch, hip, dev, gen, launches):
    """Config 3's decode step run `launches` times on the single-launch path
    with per-wave phase timestamps (100 MHz clock), each launch separately
    synchronized.  Per phase: the 10th / 50th / 90th percentile and the
    maximum over the launch's waves of (stamp - the launch's earliest start), in
    us, each the median over launches; and the share of workgroups whose XCD
    equals their index mod 8 (the round-robin dispatch the step assumes)."""
    import numpy as np

    E, H, I, topk = 64, 2048, 1536, 4
    sets = [moe_set(torch, dev, gen) for _ in range(4)]
    xs = [bf16_randn(torch, (H,), dev, gen) for _ in range(16)]
    out = torch.empty(H, dtype=torch.int16, device=dev)
    logits = torch.empty(E, dtype=torch.float32, device=dev)
    ids = torch.empty(topk, dtype=torch.int32, device=dev)
    wt = torch.empty(topk, dtype=torch.int16, device=dev)
    act = torch.empty((topk, I), dtype=torch.int16, device=dev)
    scratch = torch.zeros(hip.MOE_DECODE_SCRATCH_WORDS, dtype=torch.int32, device=dev)
    nwaves = hip.MOE_DECODE_STAMP_WAVES
    stamps = torch.zeros(nwaves * hip.MOE_DECODE_STAMPS, dtype=torch.int64, device=dev)
    per = []
    xcc_ok = []
    for i in range(launches + 3):
        g, u, d, r = sets[i % len(sets)]
        stamps.zero_()
        hip.moe_decode_stamped(r, None, g[0], u[0], d[0], E, topk, xs[i % len(xs)], out, logits, ids, wt, act,
                               scratch, stamps, mode=hip.ROUTE_SOFTMAX)
        torch.cuda.synchronize()
        if i < 3:
            continue
        st = stamps.cpu().numpy().reshape(nwaves, hip.MOE_DECODE_STAMPS)
        t0 = st[:, 0].min()
        rel = (st[:, :9].astype(np.float64) - t0) / 100.0  # 100 MHz ticks -> us
        rows = []
        for ph in range(9):
            v = rel[:, ph][st[:, ph] != 0]
            rows.append([float(np.percentile(v, 10)), float(np.percentile(v, 50)), float(np.percentile(v, 90)),
                         float(v.max())] if v.size else [float("nan")] * 4)
        per.append(rows)
        wg_xcc = st[::8, 9]  # 8 waves per workgroup
        # on the XCD of workgroup (index % 8): round-robin dispatch
        xcc_ok.append(float(np.mean(wg_xcc == wg_xcc[np.arange(256) % 8])))
    med = np.median(np.array(per), axis=0)
    del sets
    return {"phases_us_p10_p50_p90_max": {name: [round(x, 2) for x in med[i]]
                                          for i, name in enumerate(TIMELINE_PHASES)},
            "launches": launches, "xcd_round_robin_share": round(float(np.mean(xcc_ok)), 4)}


HEAD_PHASES = ("start", "loads_issued", "x_shared", "rows_stored", "keys_merged", "key_published", "collected")
HEAD8_PHASES = ("start", "x_staged", "main_loop_done", "summary_published", "finisher_words_read",
                "finisher_id_written")


def timeline_head(torch, hip, dev, gen, bits, launches, copies, batch=1):
    """The batch-1 head (65536 x 2048, Q4 or Q6, logits + argmax id) launched
    `launches` times back to back on rotating weight copies, each launch with
    per-wave phase timestamps (100 MHz clock) in a buffer of its own.  Per
    phase: the 10th / 50th / 90th percentile and maximum over the launch's
    waves of (stamp - the launch's earliest start), in us, each the median
    over launches; and per launch (medians): the waves started before the
    first workgroup finished (the first generation) and the time of the last
    of them, the time of the last start, the last workgroup key published,
    the collector's end, and the collector's end minus the last publication
    (its detection); at batch 8 the last summary published, the finisher's
    detection and its collection + recomputes, the end, and the rows the
    finisher recomputed in chunk order per batch row (median, max)."""
    import numpy as np

    n, k = 65536, 2048
    ws = make_quant(torch, n, k, bits, copies, dev, gen)
    x = bf16_randn(torch, (batch, k), dev, gen)
    y = torch.empty((batch, n), dtype=torch.int16, device=dev)
    scratch = torch.zeros(hip.argmax_scratch_words(batch), dtype=torch.int64, device=dev)
    ids = torch.empty(batch, dtype=torch.int32, device=dev)
    nw, nst = hip.GEMV_STAMP_WAVES, hip.GEMV_STAMPS
    stamps = torch.zeros((launches + 2, nw * nst), dtype=torch.int64, device=dev)
    for i in range(3):  # warm-up
        hip.gemv_quant_argmax_stamped(ws[i % copies][0], x, y, scratch, ids, stamps[0], batch)
    stamps.zero_()
    torch.cuda.synchronize()
    for i in range(launches + 2):  # back to back, as a replay runs them
        hip.gemv_quant_argmax_stamped(ws[i % copies][0], x, y, scratch, ids, stamps[i], batch)
    torch.cuda.synchronize()
    allst = stamps.cpu().numpy().reshape(launches + 2, nw, nst)[2:]
    names = HEAD_PHASES if batch == 1 else HEAD8_PHASES
    per, scal = [], []
    for st in allst:
        st = st[st[:, 0] != 0]  # the launch's waves
        t0 = st[:, 0].min()
        rel = (st[:, :len(names)].astype(np.float64) - t0) / 100.0
        rows = []
        for ph in range(len(names)):
            v = rel[:, ph][st[:, ph] != 0]
            rows.append([float(np.percentile(v, 10)), float(np.percentile(v, 50)), float(np.percentile(v, 90)),
                         float(v.max())] if v.size else [float("nan")] * 4)
        per.append(rows)
        starts = np.sort(rel[:, 0])
        if batch == 1:
            first_done = rel[:, 4][st[:, 4] != 0].min()
            gen1 = starts[starts < first_done]
            last_pub = rel[:, 5][st[:, 5] != 0].max()
            coll = rel[:, 6][st[:, 6] != 0].max()
            scal.append([gen1.size, gen1.max(), starts.max(), last_pub, coll, coll - last_pub])
        else:
            last_pub = rel[:, 3][st[:, 3] != 0].max()
            words = rel[:, 4][st[:, 4] != 0].max()
            end = rel[:, 5][st[:, 5] != 0].max()
            cand = st[st[:, 5] != 0, 6].astype(np.float64)  # the finisher waves' recomputed rows
            scal.append([len(starts), starts.max(), last_pub, words - last_pub, end - words, end,
                         float(np.median(cand)), float(cand.max())])
    med = np.median(np.array(per), axis=0)
    ms = np.median(np.array(scal), axis=0)
    del ws
    out = {"phases_us_p10_p50_p90_max": {name: [round(v, 2) for v in med[i]] for i, name in enumerate(names)}}
    if batch == 1:
        out.update(first_generation_waves=int(ms[0]), first_generation_last_start_us=round(float(ms[1]), 2),
                   last_start_us=round(float(ms[2]), 2), last_key_published_us=round(float(ms[3]), 2),
                   collector_end_us=round(float(ms[4]), 2), collector_detection_us=round(float(ms[5]), 2))
    else:
        out.update(waves_started=int(ms[0]), last_start_us=round(float(ms[1]), 2),
                   last_summary_published_us=round(float(ms[2]), 2),
                   finisher_detection_us=round(float(ms[3]), 2), finisher_collect_recompute_us=round(float(ms[4]), 2),
                   end_us=round(float(ms[5]), 2), recomputed_rows_median=float(ms[6]),
                   recomputed_rows_max=float(ms[7]))
    out.update(launches=launches)
    return out


def timeline_config4(torch, hip, dev, gen, launches):
    """Config 4's prefill step run `launches` times back to back with the two
    grouped GEMMs stamped per workgroup (start, end, block-map entry and its
    rows), replayed from a HIP graph as the bench times the step; the stamps
    are those of the sixth replay (the first ones run while the GPU's clocks
    ramp up: ~0.46 against ~0.41 ms per step).  Per GEMM (medians over
    launches): the span from the first start
    to the last end, the workgroups' busy time over span x CUs (one workgroup
    per CU at a time), the time from a workgroup's start to its entry read
    (workgroups with rows), and each workgroup's duration by its entry's
    32-row blocks (the passes: up to 8 blocks in one, 9..16 in two)."""
    import numpy as np

    E, H, I, topk, m = 64, 2048, 1536, 4, 4096
    sets = [moe_set(torch, dev, gen) for _ in range(2)]
    x = bf16_randn(torch, (m, H), dev, gen)
    out = torch.empty((m, H), dtype=torch.int16, device=dev)
    total, offs = hip.moe_prefill_workspace(m, E, topk, H, I)
    ws = torch.zeros(total, dtype=torch.uint8, device=dev)
    nst = 2 * hip.PREFILL_STAMP_WGS * hip.PREFILL_STAMPS
    stamps = torch.zeros((launches + 1, nst), dtype=torch.int64, device=dev)

    def run():
        for i in range(launches + 1):
            g, u, d, r = sets[i % len(sets)]
            hip.moe_prefill_stamped(r, None, g[0], u[0], d[0], E, topk, x, m, out, ws, total, stamps[i],
                                    mode=hip.ROUTE_SOFTMAX)

    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for _ in range(5):
        graph.replay()
    stamps.zero_()
    graph.replay()
    torch.cuda.synchronize()
    del graph
    allst = stamps.cpu().numpy().reshape(launches + 1, 2, hip.PREFILL_STAMP_WGS, hip.PREFILL_STAMPS)[1:]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    res = {}
    for gi, name in ((0, "gate_up_swiglu"), (1, "down")):
        spans, busy, by_rb, entry = [], [], {}, []
        for st in allst[:, gi]:
            st = st[st[:, 0] != 0]
            t0, t1 = st[:, 0].min(), st[:, 1].max()
            dur = (st[:, 1] - st[:, 0]) / 100.0
            spans.append((t1 - t0) / 100.0)
            busy.append(float(dur.sum() / (cus * (t1 - t0) / 100.0)))
            ent = st[:, 2] & 0xffffffff
            rows = st[:, 2] >> 32
            for rb, dv in zip(((rows + 31) // 32)[ent != 0xffffffff], dur[ent != 0xffffffff]):
                by_rb.setdefault(int(rb), []).append(float(dv))
            has = (ent != 0xffffffff) & (rows > 0)
            entry.append(float(np.median((st[has, 3] - st[has, 0]) / 100.0)))
        res[name] = {"workgroups": int((allst[0, gi][:, 0] != 0).sum()),
                     "span_us": round(float(np.median(spans)), 1), "busy_over_span": round(float(np.median(busy)), 3),
                     "entry_read_us": round(float(np.median(entry)), 2),
                     "us_by_row_blocks": {str(k): [round(float(np.median(v)), 1), len(v) // launches]
                                          for k, v in sorted(by_rb.items())}}
    del sets
    return {**res, "launches": launches, "cus": cus}


def bench_config4(torch, hip, dev, gen, steps, warmup):
    E, H, I, topk, m = 64, 2048, 1536, 4, 4096
    sets = [moe_set(torch, dev, gen) for _ in range(2)]
    x = bf16_randn(torch, (m, H), dev, gen)
    out = torch.empty((m, H), dtype=torch.int16, device=dev)
    total, offs = hip.moe_prefill_workspace(m, E, topk, H, I)
    ws = torch.zeros(total, dtype=torch.uint8, device=dev)

    def step(i):
        g, u, d, r = sets[i % len(sets)]
        hip.moe_prefill(r, None, g[0], u[0], d[0], E, topk, x, m, out, ws, total,
                        mode=hip.ROUTE_SOFTMAX)

    ms_step = timed(torch, step, max(2, steps // 4), max(1, warmup // 4))
    # the two grouped GEMMs alone, replayed on the workspace of the last step:
    # as the step runs them (the launch-ordered maps), and through the
    # reference-order entry points (each workgroup ranks the map rows)
    g, u, d, r = sets[(max(2, steps // 4) + max(1, warmup // 4) - 1) % len(sets)]
    base = ws.data_ptr()
    s = m * topk
    gu_bn, dn_bn, bm = hip.MoeTile.GU512[1], hip.MoeTile.DN512[1], hip.MoeTile.GU512[0]
    m_tiles = -(-s // bm) + E
    max_gu, max_dn = m_tiles * I // gu_bn, m_tiles * H // dn_bn
    grid_gu, grid_dn = hip.map_grid(max_gu, I // gu_bn), hip.map_grid(max_dn, H // dn_bn)

    def gemms(i):
        hip.gemm_q4_grouped_gu_act_ordered(x, base + offs["ids_sorted"], m, g[0], u[0], base + offs["act"],
                                           base + offs["gu_ord"], grid_gu, s, I, hip.MoeTile.GU512)
        hip.gemm_q4_grouped_ordered(base + offs["act"], d[0], base + offs["ed"], base + offs["dn_ord"], grid_dn,
                                    s, H, hip.MoeTile.DN512)

    def gemms_public(i):
        hip.gemm_q4_grouped_gu_act(x, base + offs["ids_sorted"], m, g[0], u[0], base + offs["act"],
                                   base + offs["gu_map"], max_gu, s, I, hip.MoeTile.GU512)
        hip.gemm_q4_grouped_mlx(base + offs["act"], d[0], base + offs["ed"], base + offs["dn_map"],
                                max_dn, s, H, hip.MoeTile.DN512)

    ms_gemm = timed(torch, gemms, max(2, steps // 4), 1)
    ms_public = timed(torch, gemms_public, max(2, steps // 4), 1)
    del sets, ws
    return ms_step, ms_gemm, ms_public


def measure_ceilings(torch, dev, steps, warmup):
    """What this part reaches with nothing but the bound resource in use
    (libmolten_ceiling.so): a streaming read of the LM heads' byte counts
    (config 2 75.6 MB, config 5 109 MB; rotated over 5 copies, as the GEMVs
    are) and of 1 GiB, and the bf16 matrix cores with independent MFMAs
    only.  The read is the best of a small sweep of launch shapes."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "molten_amd", "libmolten_ceiling.so"))
    vp, u32 = ctypes.c_void_p, ctypes.c_uint32
    lib.mhc_read.argtypes = [vp, ctypes.c_size_t, u32, u32, ctypes.c_int, vp, vp]
    lib.mhc_mfma.argtypes = [vp, u32, u32, vp]
    lib.mhc_mfma_flops.argtypes = [u32, u32]
    lib.mhc_mfma_flops.restype = ctypes.c_uint64
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    out = {}

    def stream():
        return vp(torch.cuda.current_stream().cuda_stream)

    for key, nbytes, copies in (("hbm_read_75.6MB", 75_632_640, 5), ("hbm_read_109MB", 109_187_072, 5),
                                ("hbm_read_1GiB", 1 << 30, 1)):
        bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device=dev).random_() for _ in range(copies)]
        best = None
        for unroll, grid in ((1, 2048), (1, 4096), (4, 512), (8, 256)):
            def fn(i, unroll=unroll, grid=grid):
                rc = lib.mhc_read(bufs[i % copies].data_ptr(), nbytes, grid, unroll, 1, sink.data_ptr(), stream())
                assert rc == 0, rc
            ms = timed(torch, fn, steps, warmup)
            if best is None or ms < best[0]:
                best = (ms, unroll, grid)
        ms, unroll, grid = best
        out[key] = dict(value=round(nbytes / (ms * 1e-3) / 1e9, 1), unit="GB/s", us=round(ms * 1e3, 2),
                        frac_of_hbm_peak=round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        launch=f"{grid} x 256 threads, {unroll} x 16-byte non-temporal loads in flight")
        del bufs
    fo = torch.empty(1024 * 256, dtype=torch.float32, device=dev)
    wg, iters = 512, 1000

    def mf(i):
        assert lib.mhc_mfma(fo.data_ptr(), wg, iters, stream()) == 0

    ms = timed(torch, mf, max(4, steps // 20), 2)
    tf = lib.mhc_mfma_flops(wg, iters) / (ms * 1e-3) / 1e12
    out["bf16_mfma_32x32x16"] = dict(value=round(tf, 1), unit="TFLOP/s", us=round(ms * 1e3, 1),
                                     frac_of_bf16_peak=round(tf / BF16_PEAK_TFLOPS, 4),
                                     launch=f"{wg} x 4 waves, 8 independent accumulators per wave")
    # store-to-visible latency of an 8-byte word between workgroups (the
    # fused decode step's exchanges): p50 / p90 over the consumers of 20
    # launches per mode, in ns
    import numpy as np

    lib.mhc_exchange.argtypes = [vp, vp, u32, ctypes.c_uint64, ctypes.c_int, u32, u32, vp]
    words = torch.zeros(64, dtype=torch.int64, device=dev)
    xo = torch.zeros(256 * 4, dtype=torch.int64, device=dev)
    lat = {"same_xcd_plain_store": [], "same_xcd_coherent_store": [], "cross_xcd_coherent_store": []}
    rr = []
    value = 1
    for mode in (0, 1):
        for _ in range(20):
            value += 1
            xo.zero_()
            assert lib.mhc_exchange(words.data_ptr(), xo.data_ptr(), 256, value, mode, 300, 1 << 16, stream()) == 0
            torch.cuda.synchronize()
            o = xo.cpu().numpy().reshape(256, 4)
            # same XCD as workgroup (index % 8): round-robin dispatch (the
            # XCD numbering itself need not equal index % 8)
            rr.append(float(np.mean(o[:, 0] == o[np.arange(256) % 8, 0])))
            for b in range(8, 256):
                for col, producer, key in ((1, b % 8, "same_xcd_plain_store" if mode == 0 else "same_xcd_coherent_store"),
                                           (2, (b + 1) % 8, "cross_xcd_coherent_store")):
                    if col == 2 and mode == 0:
                        continue
                    if o[b, col] != 0:
                        lat[key].append((int(o[b, col]) - int(o[producer, 3])) * 10.0)
    for key, v in lat.items():
        v = np.array(v)
        out[f"exchange_{key}"] = dict(p50_ns=round(float(np.percentile(v, 50)), 0) if v.size else None,
                                      p90_ns=round(float(np.percentile(v, 90)), 0) if v.size else None,
                                      seen=int(v.size), of=20 * 248)
    out["exchange_xcd_round_robin_share"] = round(float(np.mean(rr)), 4)
    del words, xo
    # the vendor library's bf16 GEMM (torch.bmm / torch.mm: hipBLASLt) on
    # config 4's per-expert shapes and on one dense shape, bf16 operands
    # already in memory (no dequantization, no row gather): what a plain
    # bf16 GEMM reaches at these sizes
    for key, e, m, kk, n in (("vendor_bf16_bmm_64x256x2048x3072", 64, 256, 2048, 3072),
                             ("vendor_bf16_bmm_64x256x1536x2048", 64, 256, 1536, 2048),
                             ("vendor_bf16_mm_4096x2048x11776", 1, 4096, 2048, 11776)):
        a = torch.randn(e, m, kk, device=dev, dtype=torch.bfloat16)
        b = torch.randn(e, kk, n, device=dev, dtype=torch.bfloat16)  # contiguous right operand
        c = torch.empty(e, m, n, device=dev, dtype=torch.bfloat16)
        if e == 1:
            a2, b2, c2 = a[0], b[0], c[0]
            ms = timed(torch, lambda i: torch.mm(a2, b2, out=c2), max(4, steps // 10), 2)
        else:
            ms = timed(torch, lambda i: torch.bmm(a, b, out=c), max(4, steps // 10), 2)
        tf = 2.0 * e * m * n * kk / (ms * 1e-3) / 1e12
        out[key] = dict(value=round(tf, 1), unit="TFLOP/s", us=round(ms * 1e3, 1),
                        frac_of_bf16_peak=round(tf / BF16_PEAK_TFLOPS, 4))
        del a, b, c
    return out


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _repeat(fn, budget_s: float, max_reps: int = 1000):
    """Seconds per call of fn() over about budget_s seconds (after one warm call)."""
    fn()
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= max_reps:
            return el / reps, reps, el


def cpu_baselines(budget_s: float, threads_all: int):
    """The C oracle (the same code the parity tests check against: MLX
    affine dequant semantics, f32 accumulation, OpenMP over output rows /
    expert rows) on the host cores, every BASELINE config at 1 thread and at
    `threads_all` threads, each timed for about budget_s seconds.  Config 4
    times the oracle's grouped GEMMs alone (gate, up and down of `ne`
    experts x 256 rows, the config's mean rows per expert: one expert at 1
    thread, one per thread at `threads_all`), not the router, sort and
    combine around them, and is reported in FLOP/s of those rows."""
    import numpy as np

    from molten_amd import layout
    from oracle import oracle as orc

    rng = np.random.default_rng(0)
    h4 = layout.synth_quant(rng, 65536, 2048, 4)
    h6 = layout.synth_quant(rng, 65536, 2048, 6)
    h1 = layout.synth_quant(rng, 2048, 2048, 4)
    x1 = layout.synth_bf16(rng, (1, 2048))
    x8 = layout.synth_bf16(rng, (8, 2048))
    E, H, I, topk, m = 64, 2048, 1536, 4, 4096
    gate = layout.synth_quant(rng, E * I, H, 4)
    up = layout.synth_quant(rng, E * I, H, 4)
    down = layout.synth_quant(rng, E * H, I, 4)
    router = layout.f32_to_bf16((rng.normal(0, 0.02, (E, H))).astype(np.float32))
    xm = layout.synth_bf16(rng, (m, H))

    def head(h, x, b):
        def f():
            y = orc.gemv_quant(h, x, b)
            for r in range(b):
                orc.argmax_bf16(y[r])
        return f

    out = {"cpu_model": _cpu_model(), "nproc": os.cpu_count()}
    for threads in (1, threads_all):
        orc.set_threads(threads)
        res = {}
        for key, fn, unit_work in (
                ("config1", lambda: orc.gemv_quant(h1, x1, 1), BYTES["config1"]),
                ("config2", head(h4, x1, 1), BYTES["config2"]),
                ("config5_b1", head(h6, x1, 1), BYTES["config5_b1"]),
                ("config5_b8", head(h6, x8, 8), BYTES["config5_b8"]),
                ("config3", lambda: orc.moe_decode(router, None, 1, gate, up, down, E, topk, H, I,
                                                   xm[len(res) % m]), BYTES["config3"])):
            per, reps, el = _repeat(fn, budget_s)
            res[key] = dict(value=round(unit_work / per / 1e9, 3), unit="GB/s", ms_per_step=round(per * 1e3, 3),
                            reps=reps)
        # config 4: the grouped GEMMs (gate, up, down) of `ne` experts with
        # 256 rows each (the config's mean rows per expert), one block-map
        # entry per expert covering all its columns
        ne = 1 if threads == 1 else threads
        rows = 256
        a_gu = xm[:ne * rows]
        a_dn = layout.synth_bf16(rng, (ne * rows, I))
        mg = np.array([[e * rows, e * I, 0, (e + 1) * rows] for e in range(ne)], np.uint32)
        md = np.array([[e * rows, e * H, 0, (e + 1) * rows] for e in range(ne)], np.uint32)

        def grouped():
            orc.gemm_q4_grouped(a_gu, gate, mg, ne, I, I)
            orc.gemm_q4_grouped(a_gu, up, mg, ne, I, I)
            orc.gemm_q4_grouped(a_dn, down, md, ne, H, H)

        per, reps, el = _repeat(grouped, budget_s, max_reps=50)
        flops = 3.0 * 2 * ne * rows * I * H
        res["config4"] = dict(value=round(flops / per / 1e9, 2), unit="GFLOP/s", ms_per_step=round(per * 1e3, 1),
                              reps=reps, sample=f"gate, up and down grouped GEMMs of {ne} expert(s) x {rows} rows "
                                                f"(the config's mean rows per expert); the full config is 64 experts")
        out[f"threads_{threads}"] = res
    orc.set_threads(threads_all)
    return out


def cpu_baseline_config2(budget_s: float):
    """The C oracle's Q4 LM-head GEMV (65536 x 2048, batch 1) + argmax on the
    host cores, repeated for about `budget_s` seconds."""
    import numpy as np

    from molten_amd import layout
    from oracle import oracle as orc

    rng = np.random.default_rng(0)
    h = layout.synth_quant(rng, 65536, 2048, 4)
    x = layout.synth_bf16(rng, (1, 2048))
    per, reps, el = _repeat(lambda: orc.argmax_bf16(orc.gemv_quant(h, x, 1)[0]), budget_s)
    return dict(value=round(BYTES["config2"] / per / 1e9, 3), unit="GB/s", cores=orc.get_threads(),
                kind="port",
                sample=f"full config 2 workload (65536x2048 Q4 GEMV + argmax) x {reps} reps, "
                       f"{el:.1f} s, {per * 1e3:.1f} ms per step")


def read_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprof
    PMC summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), if present."""
    p = os.path.join(ROOT, "profiles", "gemv_q4_lm_head_traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def calibrate_copy(torch, dev, mib):
    """A plain elementwise kernel (f32 negate) that reads and writes exactly
    `mib` MiB each: the scale of the PMC byte counters in the same run."""
    src = torch.ones((mib << 20) // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="time budget of the CPU baseline sample (0 = skip)")
    ap.add_argument("--cpu-all-seconds", type=float, default=1.5,
                    help="time budget of each per-config CPU baseline sample (0 = skip)")
    ap.add_argument("--only-headline", action="store_true", help="skip configs 1, 3, 4, 5")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="also run a plain elementwise copy (f32 negate) of this many MiB "
                         "(PMC byte calibration)")
    ap.add_argument("--timeline", type=int, default=0,
                    help="only print the per-phase timeline of config 3's decode step over this many "
                         "launches (device timestamps), then exit")
    ap.add_argument("--head-timeline", type=int, default=0,
                    help="only print the per-phase timelines of the heads (configs 2, 5 b=1 and 5 b=8) over "
                         "this many launches (device timestamps), then exit")
    ap.add_argument("--gemm-timeline", type=int, default=0,
                    help="only print the workgroup timelines of config 4's grouped GEMMs over this many "
                         "prefill steps (device timestamps), then exit")
    ap.add_argument("--only", choices=("config2", "config3", "config4", "config5"), default=None,
                    help="only time this workload, print its line and exit (for profiler runs)")
    ap.add_argument("--eager", action="store_true",
                    help="launch the timed steps directly instead of replaying a graph "
                         "(for counter collection; host launch overhead is then timed)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(--gpus must be 1).", file=sys.stderr)
        return 2

    import torch

    from molten_amd import hip

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    hip.load()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    steps, warmup = args.steps, args.warmup
    if args.timeline > 0:
        print(json.dumps({"timeline": "config3_moe_decode_step",
                          **timeline_config3(torch, hip, dev, gen, args.timeline)}), flush=True)
        return 0

    if args.gemm_timeline > 0:
        print(json.dumps({"timeline": "config4_grouped_gemms",
                          **timeline_config4(torch, hip, dev, gen, args.gemm_timeline)}), flush=True)
        return 0
    if args.head_timeline > 0:
        for name, bits, copies, batch in (("config2_q4_lm_head_argmax", 4, 5, 1),
                                          ("config5_b1_q6_lm_head_argmax", 6, 4, 1),
                                          ("config5_b8_q6_lm_head_argmax", 6, 4, 8)):
            print(json.dumps({"timeline": name, **timeline_head(torch, hip, dev, gen, bits, args.head_timeline,
                                                                copies, batch)}), flush=True)
        return 0

    if args.only is not None and args.calibrate_copy_mib > 0:
        calibrate_copy(torch, dev, args.calibrate_copy_mib)
    if args.only == "config4":
        ms4, ms4g, ms4p = bench_config4(torch, hip, dev, gen, steps, warmup)
        print(json.dumps({"only": "config4_prefill_moe", "ms_per_step": round(ms4, 4),
                          "grouped_gemm_only_ms": round(ms4g, 4),
                          "grouped_gemm_only_tflops": round(FLOPS_CONFIG4 / (ms4g * 1e-3) / 1e12, 2),
                          "grouped_gemm_reference_order_ms": round(ms4p, 4)}), flush=True)
        return 0
    if args.only == "config2":
        ms2 = bench_lm_head(torch, hip, dev, gen, 4, 1, steps, warmup, copies=5)
        print(json.dumps({"only": "config2_lm_head_q4_argmax", "ms_per_step": round(ms2, 5),
                          "GB/s": round(BYTES["config2"] / (ms2 * 1e-3) / 1e9, 1)}), flush=True)
        return 0
    if args.only == "config5":
        for batch in (1, 8):
            ms5 = bench_lm_head(torch, hip, dev, gen, 6, batch, steps, warmup, copies=4)
            print(json.dumps({"only": f"config5_b{batch}_q6_lm_head_argmax", "ms_per_step": round(ms5, 5),
                              "GB/s": round(BYTES[f"config5_b{batch}"] / (ms5 * 1e-3) / 1e9, 1)}), flush=True)
        return 0
    if args.only == "config3":
        ms3 = bench_config3(torch, hip, dev, gen, steps, warmup)
        print(json.dumps({"only": "config3_moe_decode_step", "ms_per_step": round(ms3, 5)}), flush=True)
        return 0

    log("config 2: Q4 LM head + argmax")
    ms2 = bench_lm_head(torch, hip, dev, gen, 4, 1, steps, warmup, copies=5)
    gbs2 = BYTES["config2"] / (ms2 * 1e-3) / 1e9
    if args.calibrate_copy_mib > 0:
        calibrate_copy(torch, dev, args.calibrate_copy_mib)
    others = {}
    if not args.only_headline:
        log("config 1: Q4 GEMV 2048x2048")
        ms1 = bench_config1(torch, hip, dev, gen, steps, warmup)
        others["config1_q4_gemv_2048"] = dict(
            value=round(BYTES["config1"] / (ms1 * 1e-3) / 1e9, 1), unit="GB/s",
            ms_per_step=round(ms1, 5), frac_of_hbm_peak=round(BYTES["config1"] / (ms1 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        log("next rows: proj3, conv3, dense down K=11776, Q6 gather, token tail, Gumbel draw, dense prefill")
        ms_p, ms_c, ms_d, ms_g, ms_t, ms_x, (ms_s, ms_kp) = bench_next_rows(torch, hip, dev, gen, steps, warmup)
        for key, n, ms in zip(("next_dense_prefill_q4_4096x2048x2048", "next_dense_prefill_q4_4096x11776x2048",
                               "next_gemm_bf16_nt_4096x2048x2048", "next_gemm_quant_bf16_nt_q4_4096x2048x2048"),
                              (2048, 11776, 2048, 2048), ms_x):
            tf = 2.0 * 4096 * n * 2048 / (ms * 1e-3) / 1e12
            others[key] = dict(
                value=round(tf, 1), unit="TFLOP/s", ms_per_step=round(ms, 5),
                frac_of_bf16_peak=round(tf / BF16_PEAK_TFLOPS, 4))
        for key, ms in (("next_proj3_gemv_scatter", ms_p), ("next_conv3_gemv", ms_c),
                        ("next_dense_down_q4_k11776", ms_d), ("next_gather_rows_q6_4096", ms_g),
                        ("next_token_tail_embed", ms_t), ("next_sample_gumbel_128000", ms_s),
                        ("next_sample_topk_topp_128000", ms_kp)):
            v = BYTES[key] / (ms * 1e-3) / 1e9
            others[key] = dict(value=round(v, 1), unit="GB/s", ms_per_step=round(ms, 5),
                               frac_of_hbm_peak=round(v / HBM_PEAK_GBS, 4))
        log("config 3: MoE decode step")
        ms3 = bench_config3(torch, hip, dev, gen, steps, warmup)
        v3 = BYTES["config3"] / (ms3 * 1e-3) / 1e9
        others["config3_moe_decode_step"] = dict(value=round(v3, 1), unit="GB/s",
                                                 ms_per_step=round(ms3, 5),
                                                 frac_of_hbm_peak=round(v3 / HBM_PEAK_GBS, 4))
        log("config 5: Q6 LM head + argmax, b=1 and b=8")
        for b, key in ((1, "config5_b1"), (8, "config5_b8")):
            # 4 x 109 MB = 437 MB: a copy is read again only after 327 MB of
            # others, beyond the 256 MB Infinity Cache
            ms5 = bench_lm_head(torch, hip, dev, gen, 6, b, steps, warmup, copies=4)
            v5 = BYTES[key] / (ms5 * 1e-3) / 1e9
            others[f"{key}_q6_lm_head_argmax"] = dict(value=round(v5, 1), unit="GB/s",
                                                      ms_per_step=round(ms5, 5),
                                                      frac_of_hbm_peak=round(v5 / HBM_PEAK_GBS, 4))
        log("config 4: prefill MoE (4096 tokens)")
        ms4, ms4g, ms4p = bench_config4(torch, hip, dev, gen, steps, warmup)
        others["config4_prefill_moe"] = dict(
            value=round(FLOPS_CONFIG4 / (ms4 * 1e-3) / 1e12, 2), unit="TFLOP/s",
            ms_per_step=round(ms4, 4),
            grouped_gemm_only_tflops=round(FLOPS_CONFIG4 / (ms4g * 1e-3) / 1e12, 2),
            grouped_gemm_only_ms=round(ms4g, 4),
            grouped_gemm_reference_order_ms=round(ms4p, 4),
            frac_of_bf16_peak=round(FLOPS_CONFIG4 / (ms4g * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4))

    log("ceilings: streaming read, bf16 matrix cores, exchange latency, the vendor bf16 GEMM")
    ceilings = measure_ceilings(torch, dev, min(steps, 100), min(warmup, 5))

    cpu = None
    if args.cpu_seconds > 0:
        log("CPU baseline (oracle, config 2)")
        cpu = cpu_baseline_config2(args.cpu_seconds)
        if not args.only_headline and args.cpu_all_seconds > 0:
            log("CPU baseline (oracle, every config, 1 thread and all threads)")
            from oracle import oracle as orc
            cpu["per_config"] = cpu_baselines(args.cpu_all_seconds, orc.get_threads())

    line = {
        "metric": "Q4 LM-head GEMV + argmax HBM GB/s (config 2; MoE decode / prefill under others)",
        "value": round(gbs2, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms2, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (BASELINE distributions, random init; weights rotated over >= 300 MB: "
                "5 copies for config 2, 4 for config 5)",
        "config": {"workload": "config2_q4_lm_head_argmax", "n": 65536, "k": 2048, "bits": 4,
                   "group_size": 64, "batch": 1, "outputs": "bf16 logits + argmax id"},
        "roofline": {"bound": "hbm", "achieved": round(gbs2, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs2 / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic()},
        "cpu_baseline": cpu,
        "others": others,
        "ceilings": ceilings,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
