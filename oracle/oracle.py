"""ctypes wrapper of the C oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product (molten_amd/).  All arrays
are numpy; bf16 values are uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")


class OrcQW(ctypes.Structure):
    _fields_ = [
        ("codes", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p),
        ("n", ctypes.c_uint32),
        ("k", ctypes.c_uint32),
        ("gs", ctypes.c_uint32),
        ("bits", ctypes.c_uint32),
    ]


_lib = None


def build() -> None:
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.orc_bf16_to_f32.restype = ctypes.c_float
        _lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.orc_expf.restype = ctypes.c_float
        _lib.orc_expf.argtypes = [ctypes.c_float]
        _lib.orc_sigmoid_max_drop.restype = ctypes.c_double
        _lib.orc_sigmoid_max_drop.argtypes = []
        _lib.orc_argmax_bf16.restype = ctypes.c_uint32
        _lib.orc_argmax_key.restype = ctypes.c_uint64
        _lib.orc_argmax_key.argtypes = [ctypes.c_float, ctypes.c_uint32]
        _lib.orc_logf.restype = ctypes.c_float
        _lib.orc_logf.argtypes = [ctypes.c_float]
        _lib.orc_gumbel.restype = ctypes.c_float
        _lib.orc_gumbel.argtypes = [ctypes.c_uint32]
        _lib.orc_sample_gumbel.restype = ctypes.c_uint64
        _lib.orc_sample_draw.restype = ctypes.c_uint64
        _lib.orc_mass_fixed.restype = ctypes.c_uint64
        _lib.orc_mass_target.restype = ctypes.c_uint64
        _lib.orc_get_threads.restype = ctypes.c_int
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def qw(h) -> OrcQW:
    """OrcQW view of a molten_amd.layout.HostQuant (arrays must stay alive)."""
    return OrcQW(h.codes.ctypes.data, h.scales.ctypes.data, h.biases.ctypes.data,
                 h.n, h.k, h.group_size, h.bits)


def set_threads(n: int) -> None:
    lib().orc_set_threads(ctypes.c_int(n))


def get_threads() -> int:
    return lib().orc_get_threads()


def bf16_to_f32(h: int) -> float:
    return lib().orc_bf16_to_f32(h)


def f32_to_bf16(f: float) -> int:
    return lib().orc_f32_to_bf16(f)


def expf(x: float) -> float:
    return lib().orc_expf(x)


def sigmoid_max_drop() -> float:
    """Largest drop of 1 / (1 + expf(-z)) below its running maximum over
    every float z in increasing order (the routing score's monotonicity
    defect)."""
    return lib().orc_sigmoid_max_drop()


def expf_array(x: np.ndarray) -> np.ndarray:
    f = lib().orc_expf
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    dtype=np.float32).reshape(np.shape(x))


def unpack(codes: np.ndarray, bits: int, n_codes: int) -> np.ndarray:
    out = np.empty(n_codes, np.uint8)
    lib().orc_unpack(_p(np.ascontiguousarray(codes, np.uint32)), ctypes.c_uint32(bits),
                     ctypes.c_size_t(n_codes), _p(out))
    return out


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    out = np.empty((q.size * bits + 31) // 32, np.uint32)
    lib().orc_pack(_p(q), ctypes.c_uint32(bits), ctypes.c_size_t(q.size), _p(out))
    return out


def dequant_bf16(h) -> np.ndarray:
    out = np.empty((h.n, h.k), np.uint16)
    w = qw(h)
    lib().orc_dequant_bf16(ctypes.byref(w), _p(out))
    return out


def gemv_quant(h, x: np.ndarray, batch: int = 1, want_f32: bool = False):
    x = np.ascontiguousarray(x, np.uint16)
    y = np.empty((batch, h.n), np.uint16)
    yf = np.empty((batch, h.n), np.float32) if want_f32 else None
    w = qw(h)
    lib().orc_gemv_quant(ctypes.byref(w), _p(x), ctypes.c_uint32(batch), _p(y), _p(yf))
    return (y, yf) if want_f32 else y


def proj3(hq, hk, hv, x: np.ndarray, max_seq: int, pos: int, v_cache: np.ndarray):
    """q, k rows and the v rows written into v_cache (updated in place)."""
    x = np.ascontiguousarray(x, np.uint16)
    assert v_cache.dtype == np.uint16 and v_cache.flags.c_contiguous
    q = np.empty(hq.n, np.uint16)
    k = np.empty(hk.n, np.uint16)
    wq, wk, wv = qw(hq), qw(hk), qw(hv)
    lib().orc_proj3(ctypes.byref(wq), ctypes.byref(wk), ctypes.byref(wv), _p(x), _p(q), _p(k),
                    _p(v_cache), ctypes.c_uint32(max_seq), ctypes.c_uint32(pos))
    return q, k


def conv3(h, x: np.ndarray, taps: np.ndarray, state: np.ndarray):
    """(out [H], new_state [2, H]) of the decode short conv."""
    x = np.ascontiguousarray(x, np.uint16)
    taps = np.ascontiguousarray(taps, np.uint16)
    state = np.ascontiguousarray(state, np.uint16)
    H = h.n // 3
    out = np.empty(H, np.uint16)
    new_state = np.empty((2, H), np.uint16)
    w = qw(h)
    lib().orc_conv3(ctypes.byref(w), _p(x), _p(taps), _p(state), _p(out), _p(new_state))
    return out, new_state


def token_tail_embed(key: int, h, w: np.ndarray, eps: float):
    """(token, x row, normed row, key after) of the decode token tail with the Q6 table h."""
    w = np.ascontiguousarray(w, np.uint16)
    best = np.array([key], np.uint64)
    tok = np.zeros(1, np.uint32)
    x = np.empty(h.k, np.uint16)
    normed = np.empty(h.k, np.uint16)
    e = qw(h)
    lib().orc_token_tail_embed(_p(best), _p(tok), ctypes.byref(e), _p(w), _p(x), _p(normed),
                               ctypes.c_float(eps))
    return int(tok[0]), x, normed, int(best[0])


def philox(ctr, key) -> np.ndarray:
    c = np.array(ctr, np.uint32)
    k = np.array(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib().orc_philox(_p(c), _p(k), _p(out))
    return out


def logf(x: float) -> float:
    return lib().orc_logf(ctypes.c_float(x))


def gumbel(x: int) -> float:
    return lib().orc_gumbel(ctypes.c_uint32(x))


def sample_gumbel(logits: np.ndarray, seen, inv_temp: float, penalty: float, use_penalty: bool,
                  seed: int, pos: int, best: int = 0) -> int:
    """The key of the temperature-only draw (lfm_sample_gumbel), folded with best."""
    logits = np.ascontiguousarray(logits, np.uint16)
    seen = None if seen is None else np.ascontiguousarray(seen, np.uint32)
    inv_pen = np.float32(1.0) / np.float32(penalty)
    return int(lib().orc_sample_gumbel(_p(logits), ctypes.c_uint32(logits.size), _p(seen),
                                       ctypes.c_float(inv_temp), ctypes.c_float(penalty),
                                       ctypes.c_float(inv_pen), ctypes.c_int(int(use_penalty)),
                                       ctypes.c_uint32(seed & 0xffffffff), ctypes.c_uint32(seed >> 32),
                                       ctypes.c_uint32(pos), ctypes.c_uint64(best)))


def mass_fixed(w: float, m: float) -> int:
    return int(lib().orc_mass_fixed(ctypes.c_float(w), ctypes.c_float(m)))


def mass_target(z: int, top_p: float) -> int:
    return int(lib().orc_mass_target(ctypes.c_uint64(z), ctypes.c_float(top_p)))


def sample_draw(logits: np.ndarray, seen, inv_temp: float, penalty: float, use_penalty: bool, top_k: int,
                top_p: float, seed: int, pos: int, best: int = 0):
    """The kept-set draw (top-k / top-p): returns (key folded with best, tau's orderable key)."""
    logits = np.ascontiguousarray(logits, np.uint16)
    seen = None if seen is None else np.ascontiguousarray(seen, np.uint32)
    inv_pen = np.float32(1.0) / np.float32(penalty)
    tau = ctypes.c_uint32(0)
    k = lib().orc_sample_draw(_p(logits), ctypes.c_uint32(logits.size), _p(seen), ctypes.c_float(inv_temp),
                              ctypes.c_float(penalty), ctypes.c_float(inv_pen), ctypes.c_int(int(use_penalty)),
                              ctypes.c_uint32(top_k), ctypes.c_float(top_p), ctypes.c_uint32(seed & 0xffffffff),
                              ctypes.c_uint32(seed >> 32), ctypes.c_uint32(pos), ctypes.c_uint64(best),
                              ctypes.byref(tau))
    return int(k), int(tau.value)


def gemv_quant_rows(h, x: np.ndarray, rows: np.ndarray, batch: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    rows = np.ascontiguousarray(rows, np.uint32)
    y = np.empty((batch, rows.size), np.uint16)
    w = qw(h)
    lib().orc_gemv_quant_rows(ctypes.byref(w), _p(x), ctypes.c_uint32(batch), _p(rows),
                              ctypes.c_uint32(rows.size), _p(y))
    return y


def argmax_bf16(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.uint16)
    return int(lib().orc_argmax_bf16(_p(x), ctypes.c_size_t(x.size)))


def argmax_key(v: float, i: int) -> int:
    return int(lib().orc_argmax_key(v, i))


def gemv_dense(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """w: float32 [n, k] or uint16 (bf16) [n, k]; x: bf16 [m, k] -> f32 [m, n]."""
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, np.uint16).reshape(-1, w.shape[1])
    m, (n, k) = x.shape[0], w.shape
    y = np.empty((m, n), np.float32)
    lib().orc_gemv_dense(_p(w), ctypes.c_int(1 if w.dtype == np.float32 else 0), _p(x),
                         ctypes.c_uint32(m), ctypes.c_uint32(n), ctypes.c_uint32(k), _p(y))
    return y


def route(logits: np.ndarray, bias, topk: int, mode: int, eps: float = 1e-6):
    logits = np.ascontiguousarray(logits, np.float32)
    m, e = logits.reshape(-1, logits.shape[-1]).shape
    ids = np.empty((m, topk), np.uint32)
    w = np.empty((m, topk), np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_route(_p(logits), _p(b), ctypes.c_uint32(m), ctypes.c_uint32(e),
                    ctypes.c_uint32(topk), ctypes.c_int(mode), ctypes.c_float(eps), _p(ids), _p(w))
    return ids, w


def gather_act(gate, up, n_inter: int, x: np.ndarray, ids) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    slots = 1 if ids is None else len(ids)
    act = np.empty((slots, n_inter), np.uint16)
    i = None if ids is None else np.ascontiguousarray(ids, np.uint32)
    g, u = qw(gate), qw(up)
    lib().orc_gather_act(ctypes.byref(g), ctypes.byref(u), ctypes.c_uint32(n_inter), _p(x), _p(i),
                         ctypes.c_uint32(slots), _p(act))
    return act


def down_combine(down, n_out: int, act: np.ndarray, ids, w) -> np.ndarray:
    act = np.ascontiguousarray(act, np.uint16)
    ids = np.ascontiguousarray(ids, np.uint32)
    w = np.ascontiguousarray(w, np.uint16)
    out = np.empty(n_out, np.uint16)
    d = qw(down)
    lib().orc_down_combine(ctypes.byref(d), ctypes.c_uint32(n_out), _p(act), _p(ids), _p(w),
                           ctypes.c_uint32(ids.size), _p(out))
    return out


def moe_decode(router, bias, mode, gate, up, down, n_experts, topk, d_model, n_inter, x,
               eps: float = 1e-6):
    router = np.ascontiguousarray(router)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    x = np.ascontiguousarray(x, np.uint16)
    out = np.empty(d_model, np.uint16)
    logits = np.empty(n_experts, np.float32)
    ids = np.empty(topk, np.uint32)
    w = np.empty(topk, np.uint16)
    act = np.empty((topk, n_inter), np.uint16)
    g, u, d = qw(gate), qw(up), qw(down)
    lib().orc_moe_decode(_p(router), ctypes.c_int(1 if router.dtype == np.float32 else 0), _p(b),
                         ctypes.c_int(mode), ctypes.c_float(eps), ctypes.byref(g), ctypes.byref(u),
                         ctypes.byref(d), ctypes.c_uint32(n_experts), ctypes.c_uint32(topk),
                         ctypes.c_uint32(d_model), ctypes.c_uint32(n_inter), _p(x), _p(out),
                         _p(logits), _p(ids), _p(w), _p(act))
    return dict(out=out, logits=logits, ids=ids, w=w, act=act)


def moe_count(ids: np.ndarray, e: int) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.uint32).ravel()
    counts = np.empty(e, np.uint32)
    lib().orc_moe_count(_p(ids), ctypes.c_uint32(ids.size), ctypes.c_uint32(e), _p(counts))
    return counts


def moe_offsets(counts: np.ndarray) -> np.ndarray:
    counts = np.ascontiguousarray(counts, np.uint32)
    off = np.empty_like(counts)
    lib().orc_moe_offsets(_p(counts), ctypes.c_uint32(counts.size), _p(off))
    return off


def moe_sorted(ids: np.ndarray, offsets: np.ndarray, m: int, e: int, topk: int):
    ids = np.ascontiguousarray(ids, np.uint32).ravel()
    offsets = np.ascontiguousarray(offsets, np.uint32)
    ids_sorted = np.empty(m * topk, np.uint32)
    slotpos = np.empty(m * topk, np.uint32)
    lib().orc_moe_sorted(_p(ids), _p(offsets), ctypes.c_uint32(m), ctypes.c_uint32(e),
                         ctypes.c_uint32(topk), _p(ids_sorted), _p(slotpos))
    return ids_sorted, slotpos


def moe_block_offsets(counts, bm, gu_bn, dn_bn, gu_n, dn_n):
    counts = np.ascontiguousarray(counts, np.uint32)
    gu_off = np.empty_like(counts)
    dn_off = np.empty_like(counts)
    lib().orc_moe_block_offsets(_p(counts), ctypes.c_uint32(counts.size), ctypes.c_uint32(bm),
                                ctypes.c_uint32(gu_bn), ctypes.c_uint32(dn_bn),
                                ctypes.c_uint32(gu_n), ctypes.c_uint32(dn_n), _p(gu_off),
                                _p(dn_off))
    return gu_off, dn_off


def moe_blocks(counts, offsets, gu_off, dn_off, bm, gu_bn, dn_bn, gu_n, dn_n, max_gu, max_dn):
    c = [np.ascontiguousarray(a, np.uint32) for a in (counts, offsets, gu_off, dn_off)]
    gu = np.empty((max_gu, 4), np.uint32)
    dn = np.empty((max_dn, 4), np.uint32)
    lib().orc_moe_blocks(_p(c[0]), _p(c[1]), _p(c[2]), _p(c[3]), ctypes.c_uint32(c[0].size),
                         ctypes.c_uint32(bm), ctypes.c_uint32(gu_bn), ctypes.c_uint32(dn_bn),
                         ctypes.c_uint32(gu_n), ctypes.c_uint32(dn_n), _p(gu),
                         ctypes.c_uint32(max_gu), _p(dn), ctypes.c_uint32(max_dn))
    return gu, dn


def gather_rows_bf16(table: np.ndarray, ids: np.ndarray) -> np.ndarray:
    table = np.ascontiguousarray(table, np.uint16)
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.empty((ids.size, table.shape[1]), np.uint16)
    lib().orc_gather_rows_bf16(_p(table), _p(ids), ctypes.c_uint32(ids.size),
                               ctypes.c_uint32(table.shape[1]), _p(out))
    return out


def silu_mul_bf16(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, np.uint16)
    up = np.ascontiguousarray(up, np.uint16)
    out = np.empty_like(gate)
    lib().orc_silu_mul_bf16(_p(gate), _p(up), ctypes.c_size_t(gate.size), _p(out))
    return out


def moe_combine_rows(sorted_rows, slotpos, w, m, topk) -> np.ndarray:
    s = np.ascontiguousarray(sorted_rows, np.uint16)
    sp = np.ascontiguousarray(slotpos, np.uint32)
    w = np.ascontiguousarray(w, np.uint16)
    h = s.shape[1]
    out = np.empty((m, h), np.uint16)
    lib().orc_moe_combine_rows(_p(s), _p(sp), _p(w), ctypes.c_uint32(m), ctypes.c_uint32(h),
                               ctypes.c_uint32(topk), _p(out))
    return out


def gemm_q4_grouped(a: np.ndarray, h, blocks: np.ndarray, n_blocks: int, n: int, bn: int,
                    out: np.ndarray | None = None) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint16)
    c = np.zeros((a.shape[0], n), np.uint16) if out is None else out
    blocks = np.ascontiguousarray(blocks, np.uint32)
    w = qw(h)
    lib().orc_gemm_q4_grouped(_p(a), ctypes.byref(w), _p(c), _p(blocks), ctypes.c_uint32(n_blocks),
                              ctypes.c_uint32(n), ctypes.c_uint32(bn))
    return c


def moe_prefill(router, bias, mode, gate, up, down, n_experts, topk, d_model, n_inter, x,
                eps: float = 1e-6, token_mask=None):
    router = np.ascontiguousarray(router)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    x = np.ascontiguousarray(x, np.uint16)
    m = x.shape[0]
    s = m * topk
    r = dict(
        out=np.empty((m, d_model), np.uint16), ids=np.empty((m, topk), np.uint32),
        gw=np.empty((m, topk), np.uint16), counts=np.empty(n_experts, np.uint32),
        offsets=np.empty(n_experts, np.uint32), ids_sorted=np.empty(s, np.uint32),
        slotpos=np.empty(s, np.uint32), act=np.empty((s, n_inter), np.uint16),
        ed=np.empty((s, d_model), np.uint16),
    )
    g, u, d = qw(gate), qw(up), qw(down)
    mask = None if token_mask is None else np.ascontiguousarray(token_mask, np.uint8)
    lib().orc_moe_prefill_masked(_p(router), ctypes.c_int(1 if router.dtype == np.float32 else 0),
                          _p(b),
                          ctypes.c_int(mode), ctypes.c_float(eps), ctypes.byref(g), ctypes.byref(u),
                          ctypes.byref(d), ctypes.c_uint32(n_experts), ctypes.c_uint32(topk),
                          ctypes.c_uint32(d_model), ctypes.c_uint32(n_inter), ctypes.c_uint32(m),
                          _p(x), _p(mask), _p(r["out"]), _p(r["ids"]), _p(r["gw"]), _p(r["counts"]),
                          _p(r["offsets"]), _p(r["ids_sorted"]), _p(r["slotpos"]), _p(r["act"]),
                          _p(r["ed"]))
    return r
