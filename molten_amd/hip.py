"""ctypes binding of libmolten_hip.so: the operator layer of molten's hot path.

Each function mirrors one operator wrapper of the reference's Rust layer
(src/kernels/lfm.rs, src/kernels/quant.rs, src/kernels/elementwise.rs): same
name, same argument order and meaning, and it raises `MoltenError` where the
reference's `ensure!` would return an error.  Tensors are torch tensors on
the GPU (only their device pointers cross the C ABI) or plain integer device
addresses.  This is the Python counterpart of a Rust `src/hip.rs` binding
(extern "C" declarations of the same functions).

The library must be built (molten_amd/libmolten_hip.so); importing this
module without it raises: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmolten_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "molten_hip.h")


class MoltenError(RuntimeError):
    def __init__(self, code: int, op: str, msg: str):
        super().__init__(f"{op} failed ({code}): {msg}")
        self.code = code
        self.op = op


MH_OK = 0
ROUTE_SIGMOID_BIAS = 0
ROUTE_SOFTMAX = 1
DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_U32 = 2
DTYPE_OTHER = 3
MH_ERR_INVALID = -1
MH_ERR_ALIGN = -2
MH_ERR_UNSUPPORTED = -3


class CQuantWeights(ctypes.Structure):
    _fields_ = [
        ("codes", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p),
        ("out_features", ctypes.c_uint32),
        ("in_features", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
        ("bits", ctypes.c_uint32),
    ]


_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_qw = ctypes.POINTER(CQuantWeights)

# name -> argtypes; every function returns int (status) unless listed in _RESTYPES.
_SIGNATURES = {
    "mh_last_error": [],
    "mh_version": [],
    "mh_device_count": [ctypes.POINTER(ctypes.c_int)],
    "mh_set_device": [_i32],
    "mh_stream_create": [ctypes.POINTER(_vp)],
    "mh_stream_destroy": [_vp],
    "mh_stream_synchronize": [_vp],
    "mh_event_create": [ctypes.POINTER(_vp)],
    "mh_event_destroy": [_vp],
    "mh_event_record": [_vp, _vp],
    "mh_event_synchronize": [_vp],
    "mh_malloc": [ctypes.POINTER(_vp), _sz],
    "mh_free": [_vp],
    "mh_memcpy": [_vp, _vp, _sz, _i32, _vp],
    "mh_zero": [_vp, _sz, _vp],
    "mh_status": [ctypes.POINTER(_u32), _i32, _vp],
    "mh_dequant_to_bf16": [_qw, _vp, _vp],
    "mh_dequant_q4_bf16_bulk": [_qw, _vp, _vp],
    "mh_gemv_quant": [_qw, _vp, _vp, _u32, _vp],
    "mh_gemv_head_argmax": [_qw, _vp, _vp, _u32, _vp],
    "mh_gemv_quant_argmax": [_qw, _vp, _vp, _vp, _vp, _u32, _vp],
    "mh_gemv_quant_argmax_stamped": [_qw, _vp, _vp, _vp, _vp, _u32, _vp, _vp],
    "mh_gemv_quant_argmax_noalloc": [_qw, _vp, _vp, _vp, _u32, _vp],
    "mh_proj3_gemv_scatter": [_qw, _qw, _qw, _vp, _vp, _vp, _vp, _u32, _u32, _vp],
    "mh_conv3_gemv": [_qw, _vp, _vp, _vp, _vp, _vp, _vp],
    "mh_token_tail": [_vp, _vp, _u32, _vp],
    "mh_sample_gumbel": [_vp, _u32, _vp, _vp, _vp, _vp],
    "mh_sample_workspace_bytes": [_u32],
    "mh_sample_draw": [_vp, _u32, _vp, _vp, _vp, _vp, _sz, _vp],
    "mh_sample_mark": [_vp, _vp, _u32, _vp],
    "mh_checkpoint_open": [ctypes.c_char_p, ctypes.POINTER(_vp)],
    "mh_checkpoint_close": [_vp],
    "mh_checkpoint_count": [_vp],
    "mh_checkpoint_name": [_vp, _u32],
    "mh_checkpoint_meta": [_vp, ctypes.c_char_p, _vp],
    "mh_checkpoint_read": [_vp, ctypes.c_char_p, _vp, _sz, _vp],
    "mh_load_quant": [_vp, ctypes.c_char_p, _u32, _u32, _u32, _vp, _vp, _vp, _qw, _vp],
    "mh_gemm_q4_dense": [_vp, _u32, _qw, _vp, _vp],
    "mh_gemm_bf16_nt": [_vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "mh_gemm_quant_bf16_nt": [_vp, _u32, _qw, _vp, _vp, _sz, _vp],
    "mh_token_tail_embed": [_vp, _vp, _qw, _vp, _vp, _vp, _f32, _vp],
    "mh_gather_rows_q6": [_qw, _vp, _u32, _vp, _vp],
    "mh_argmax_bf16": [_vp, _u32, _vp, _vp, _vp],
    "mh_gemv_f32": [_vp, _vp, _vp, _u32, _u32, _vp],
    "mh_gemv_bf16": [_vp, _vp, _vp, _u32, _u32, _vp],
    "mh_route_token": [_vp, _vp, _vp, _vp, _u32, _u32, _i32, _f32, _vp],
    "mh_router_route": [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _i32, _f32,
                        _vp],
    "mh_gemv_gather_act": [_qw, _qw, _vp, _vp, _vp, _u32, _u32, _vp],
    "mh_gemv_gu_act": [_qw, _qw, _vp, _vp, _vp],
    "mh_gemv_gather_down_combine": [_qw, _vp, _vp, _vp, _vp, _u32, _u32, _vp],
    "mh_moe_decode": [_vp, _i32, _vp, _i32, _f32, _qw, _qw, _qw, _u32, _u32, _vp, _vp, _vp, _vp,
                      _vp, _vp, _vp, _vp],
    "mh_moe_decode_stamped": [_vp, _i32, _vp, _i32, _f32, _qw, _qw, _qw, _u32, _u32, _vp, _vp, _vp, _vp,
                              _vp, _vp, _vp, _vp, _vp],
    "mh_router_prefill": [_vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp],
    "mh_moe_route_batch": [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _i32, _f32, _vp],
    "mh_moe_zero_counts": [_vp, _u32, _vp],
    "mh_moe_count_slots": [_vp, _vp, _u32, _u32, _vp],
    "mh_moe_offsets": [_vp, _vp, _u32, _vp],
    "mh_moe_sorted": [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "mh_moe_zero_blocks": [_vp, _vp, _u32, _u32, _vp],
    "mh_moe_block_offsets": [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp],
    "mh_moe_blocks": [_vp, _vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32, _u32, _u32,
                      _u32, _vp],
    "mh_gather_rows_bf16": [_vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "mh_silu_mul_bf16": [_vp, _vp, _vp, _sz, _vp],
    "mh_moe_combine_rows": [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "mh_gemm_q4_grouped": [_vp, _qw, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp],
    "mh_gemm_q4_grouped_gu": [_vp, _qw, _qw, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp],
    "mh_gemm_q4_grouped_gu_act": [_vp, _vp, _u32, _qw, _qw, _vp, _vp, _u32, _u32, _u32, _u32,
                                  _u32, _vp],
    "mh_gemm_q4_grouped_ordered": [_vp, _qw, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp],
    "mh_gemm_q4_grouped_gu_act_ordered": [_vp, _vp, _u32, _qw, _qw, _vp, _vp, _u32, _u32, _u32, _u32,
                                          _u32, _vp],
    "mh_moe_prefill_workspace": [_u32, _u32, _u32, _u32, _u32, ctypes.POINTER(_sz)],
    "mh_moe_prefill": [_vp, _i32, _vp, _i32, _f32, _qw, _qw, _qw, _u32, _u32, _vp, _u32, _vp,
                       _vp, _sz, _vp],
    "mh_moe_prefill_stamped": [_vp, _i32, _vp, _i32, _f32, _qw, _qw, _qw, _u32, _u32, _vp, _u32, _vp,
                               _vp, _sz, _vp, _vp],
}
_RESTYPES = {"mh_last_error": ctypes.c_char_p, "mh_version": ctypes.c_char_p,
             "mh_moe_prefill_workspace": ctypes.c_size_t, "mh_sample_workspace_bytes": ctypes.c_size_t, "mh_checkpoint_close": None,
             "mh_checkpoint_count": ctypes.c_uint32, "mh_checkpoint_name": ctypes.c_char_p}

_lib: Optional[ctypes.CDLL] = None


def _one_runtime() -> None:
    """Load torch's HIP runtime first when torch is installed.

    torch ships its own libamdhip64.so with the same soname
    (libamdhip64.so.7) as the ROCm copy this library is linked against.  The
    dynamic linker resolves a DT_NEEDED entry against the sonames of the
    objects already loaded, so with torch imported first the library binds
    to torch's runtime and the process holds one HIP runtime, whose streams
    torch hands to the launchers.  Loaded the other way round, the process
    would hold two runtimes, and a stream or event of one passed to the
    other.  Without torch (the Rust host, a torch-free worker) the library
    loads the ROCm runtime on its own: again one runtime."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def hip_runtimes() -> list[str]:
    """Paths of the HIP runtime libraries mapped into this process."""
    with open("/proc/self/maps") as f:
        return sorted({ln.split()[-1] for ln in f if "libamdhip64" in ln and "/" in ln})


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the native library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')"
        )
    _one_runtime()
    lib = ctypes.CDLL(path)
    if len(hip_runtimes()) != 1:
        raise ImportError(f"{path}: more than one HIP runtime in the process: {hip_runtimes()}")
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES[name] if name in _RESTYPES else ctypes.c_int
    _lib = lib
    return lib


def declared_functions(header: str = HEADER_PATH) -> list[str]:
    """Names of every function the C header declares."""
    import re

    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mh_[a-z0-9_]+)\s*\(", text)))


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    try:
        import torch

        if torch.cuda.is_available():
            return torch.cuda.current_stream().cuda_stream
    except Exception:  # pragma: no cover - torch import failure
        pass
    return None


STATUS_ARGMAX_WAIT = 1
STATUS_DECODE_WAIT = 2


def device_status(clear: bool = True, stream=None) -> int:
    """The device status word (MH_STATUS_* bits): waits for the stream, reads
    the word and (clear) resets it."""
    v = _u32()
    check(load().mh_status(ctypes.byref(v), 1 if clear else 0, _stream(stream)), "status")
    return v.value


def check(rc: int, op: str) -> None:
    if rc != MH_OK:
        msg = load().mh_last_error().decode(errors="replace")
        raise MoltenError(rc, op, msg)


@dataclass
class QuantWeights:
    """molten's QuantWeights (src/weights.rs:11-30) over device tensors.

    codes U32 [out, in*bits/32], scales/biases bf16 [out, in/group_size]
    (any tensor dtype of the right byte size; only pointers are used)."""

    codes: object
    scales: object
    biases: object
    out_features: int
    in_features: int
    group_size: int = 64
    bits: int = 4

    def c(self) -> CQuantWeights:
        return CQuantWeights(
            _ptr(self.codes), _ptr(self.scales), _ptr(self.biases),
            self.out_features, self.in_features, self.group_size, self.bits,
        )


def _qref(w: QuantWeights):
    return ctypes.byref(w.c())


# ---------------------------------------------------------------- dequant --

def dequant_to_bf16(w: QuantWeights, out, stream=None) -> None:
    """src/kernels/quant.rs:69."""
    check(load().mh_dequant_to_bf16(_qref(w), _ptr(out), _stream(stream)), "dequant_to_bf16")


def dequant_q4_bf16_bulk(w: QuantWeights, out, stream=None) -> None:
    """src/kernels/quant.rs:95."""
    check(load().mh_dequant_q4_bf16_bulk(_qref(w), _ptr(out), _stream(stream)),
          "dequant_q4_bf16_bulk")


# ------------------------------------------------------------------ GEMVs --

def gemv_quant_argmax_noalloc(w: "QuantWeights", x, y, ids, batch: int = 1, stream=None) -> None:
    """gemv_quant_argmax with the library's own per-device finisher scratch
    (no device memory is allocated; batch 1..8)."""
    check(load().mh_gemv_quant_argmax_noalloc(_qref(w), _ptr(x), _ptr(y), _ptr(ids), batch, _stream(stream)),
          "gemv_quant_argmax_noalloc")


def gemv_quant(w: QuantWeights, x, y, batch: int = 1, stream=None) -> None:
    """src/kernels/lfm.rs:112 (batch > 1 is this build's extension)."""
    check(load().mh_gemv_quant(_qref(w), _ptr(x), _ptr(y), batch, _stream(stream)), "gemv_quant")


def gemv_head_argmax(w: QuantWeights, x, best, batch: int = 1, stream=None) -> None:
    """src/kernels/lfm.rs:826."""
    check(load().mh_gemv_head_argmax(_qref(w), _ptr(x), _ptr(best), batch, _stream(stream)),
          "gemv_head_argmax")


ARGMAX_SLOTS = 2048
MOE_DECODE_SCRATCH_WORDS = 10240  # MH_MOE_DECODE_SCRATCH_WORDS


def argmax_scratch_words(batch: int) -> int:
    """MH_ARGMAX_SCRATCH_WORDS(batch): u64 words of gemv_quant_argmax scratch."""
    return ARGMAX_SLOTS * batch + 1


def gemv_quant_argmax(w: QuantWeights, x, y, scratch, ids, batch: int = 1, stream=None) -> None:
    """Stored logits (y may be None) + argmax ids in one launch (BASELINE
    configs 2 and 5).  scratch: zeroed u64 [argmax_scratch_words(batch)]."""
    check(load().mh_gemv_quant_argmax(_qref(w), _ptr(x), _ptr(y), _ptr(scratch), _ptr(ids), batch,
                                      _stream(stream)), "gemv_quant_argmax")


GEMV_STAMP_WAVES = 8192  # MH_GEMV_STAMP_WAVES
GEMV_STAMPS = 8  # MH_GEMV_STAMPS


def gemv_quant_argmax_stamped(w: QuantWeights, x, y, scratch, ids, stamps, batch: int = 1, stream=None) -> None:
    """gemv_quant_argmax at batch 1 or 8 with per-wave phase timestamps
    (measurement only): stamps u64 [GEMV_STAMP_WAVES * GEMV_STAMPS]."""
    check(load().mh_gemv_quant_argmax_stamped(_qref(w), _ptr(x), _ptr(y), _ptr(scratch), _ptr(ids), batch,
                                              _ptr(stamps), _stream(stream)), "gemv_quant_argmax_stamped")


def token_tail(best, out_tok, batch: int = 1, stream=None) -> None:
    """src/kernels/lfm.rs:850 without `next`."""
    check(load().mh_token_tail(_ptr(best), _ptr(out_tok), batch, _stream(stream)), "token_tail")


def argmax_bf16(x, n: int, partials, out, stream=None) -> None:
    """src/kernels/lfm.rs:794."""
    check(load().mh_argmax_bf16(_ptr(x), n, _ptr(partials), _ptr(out), _stream(stream)),
          "argmax_bf16")


def zero(buf, nbytes: int, stream=None) -> None:
    check(load().mh_zero(_ptr(buf), nbytes, _stream(stream)), "zero")


def _dtype_of(w) -> int:
    """MH_DTYPE_* of a router tensor (torch f32 -> F32, 2-byte -> BF16)."""
    es = w.element_size() if hasattr(w, "element_size") else w.itemsize
    return DTYPE_F32 if es == 4 else DTYPE_BF16


# ----------------------------------------------------------- router / MoE --

def gemv_f32(w, x, y, n: int, k: int, stream=None) -> None:
    """src/kernels/lfm.rs:314 (f32 router)."""
    check(load().mh_gemv_f32(_ptr(w), _ptr(x), _ptr(y), n, k, _stream(stream)), "gemv_f32")


def gemv_bf16(w, x, y, n: int, k: int, stream=None) -> None:
    """bf16-router counterpart of gemv_f32."""
    check(load().mh_gemv_bf16(_ptr(w), _ptr(x), _ptr(y), n, k, _stream(stream)), "gemv_bf16")


def route_token(logits, bias, ids, weights, e: int, topk: int, mode: int = ROUTE_SIGMOID_BIAS,
                eps: float = 1e-6, stream=None) -> None:
    """src/kernels/lfm.rs:391."""
    check(load().mh_route_token(_ptr(logits), _ptr(bias), _ptr(ids), _ptr(weights), e, topk, mode,
                                eps, _stream(stream)), "route_token")


def router_route(w, x, logits, bias, ids, weights, counter, e: int, k: int, topk: int,
                 mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """src/kernels/lfm.rs:266 without the add+RMSNorm prologue."""
    check(load().mh_router_route(_ptr(w), _dtype_of(w), _ptr(x), _ptr(logits), _ptr(bias),
                                 _ptr(ids), _ptr(weights), _ptr(counter), e, k, topk, mode, eps,
                                 _stream(stream)), "router_route")


def proj3_gemv_scatter(q: QuantWeights, k: QuantWeights, v: QuantWeights, x, q_out, k_out, v_cache,
                       max_seq: int, pos: int, stream=None) -> None:
    """src/kernels/lfm.rs:155 (q_out, k_out stored; V rows into v_cache at pos)."""
    check(load().mh_proj3_gemv_scatter(_qref(q), _qref(k), _qref(v), _ptr(x), _ptr(q_out),
                                       _ptr(k_out), _ptr(v_cache), max_seq, pos, _stream(stream)),
          "proj3_gemv_scatter")


def conv3_gemv(wproj: QuantWeights, x, taps, state, out, new_state, stream=None) -> None:
    """src/kernels/lfm.rs:220 (the decode short conv with its input projection)."""
    check(load().mh_conv3_gemv(_qref(wproj), _ptr(x), _ptr(taps), _ptr(state), _ptr(out),
                               _ptr(new_state), _stream(stream)), "conv3_gemv")


def token_tail_embed(best, out_tok, table: QuantWeights, w, x, normed, eps: float,
                     stream=None) -> None:
    """src/kernels/lfm.rs:850 token_tail with `next` (the token's embedding row + RMSNorm)."""
    check(load().mh_token_tail_embed(_ptr(best), _ptr(out_tok), _qref(table), _ptr(w), _ptr(x),
                                     _ptr(normed), eps, _stream(stream)), "token_tail_embed")


def gather_rows_q6(table: QuantWeights, ids, m: int, out, stream=None) -> None:
    """src/kernels/lfm.rs:337 (dequantizing embedding gather)."""
    check(load().mh_gather_rows_q6(_qref(table), _ptr(ids), m, _ptr(out), _stream(stream)),
          "gather_rows_q6")


def gemm_q4_dense(a, m: int, w: QuantWeights, c, stream=None) -> None:
    """src/lfm.rs:661 (prefill dense projection: dequant + bf16 GEMM, fused)."""
    check(load().mh_gemm_q4_dense(_ptr(a), m, _qref(w), _ptr(c), _stream(stream)), "gemm_q4_dense")


def gemm_bf16_nt(a, b, c, m: int, n: int, k: int, stream=None) -> None:
    """src/kernels/gemm.rs:33: C[m, n] = A[m, k] . B[n, k]^T (bf16, f32 accumulation)."""
    check(load().mh_gemm_bf16_nt(_ptr(a), _ptr(b), _ptr(c), m, n, k, _stream(stream)), "gemm_bf16_nt")


def gemm_quant_bf16_nt(a, m: int, w: QuantWeights, c, scratch, scratch_elems: int, stream=None) -> None:
    """src/kernels/quant.rs:126: W dequantized into scratch, then gemm_bf16_nt."""
    check(load().mh_gemm_quant_bf16_nt(_ptr(a), m, _qref(w), _ptr(c), _ptr(scratch), scratch_elems,
                                       _stream(stream)), "gemm_quant_bf16_nt")


class SampleParams(ctypes.Structure):
    """The reference's SmpParams head (src/lfm/sample.rs:175-192)."""
    _fields_ = [("inv_temp", ctypes.c_float), ("penalty", ctypes.c_float), ("inv_penalty", ctypes.c_float),
                ("use_penalty", ctypes.c_uint32), ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float),
                ("seed_lo", ctypes.c_uint32), ("seed_hi", ctypes.c_uint32), ("pos", ctypes.c_uint32),
                ("pad0", ctypes.c_uint32)]


def sample_params(temperature: float, seed: int, pos: int, penalty: float = 1.0, top_k: int = 0,
                  top_p: float = 1.0) -> SampleParams:
    import numpy as np
    return SampleParams(float(np.float32(1.0) / np.float32(temperature)), penalty,
                        float(np.float32(1.0) / np.float32(penalty)), int(penalty != 1.0), top_k, top_p,
                        seed & 0xffffffff, seed >> 32, pos, 0)


def sample_gumbel(logits, n: int, seen, params: SampleParams, best, stream=None) -> None:
    """src/lfm/sample.rs:264 encode_draw, temperature only (the key folds into best)."""
    check(load().mh_sample_gumbel(_ptr(logits), n, _ptr(seen), ctypes.byref(params), _ptr(best),
                                  _stream(stream)), "sample_gumbel")


SAMPLE_ZERO_BYTES = 16640  # MH_SAMPLE_ZERO_BYTES: the kept-set workspace's head that must start zero


def sample_workspace_bytes(n: int) -> int:
    """mh_sample_workspace_bytes: the kept-set draw's workspace for a vocabulary of n."""
    return int(load().mh_sample_workspace_bytes(n))


def sample_draw(logits, n: int, seen, params: SampleParams, best, workspace, workspace_bytes: int,
                stream=None) -> None:
    """src/lfm/sample.rs:264-330 encode_draw, every case: top-k / top-p kept set
    (exact thresholds) and the Gumbel-max over it, folded into best."""
    check(load().mh_sample_draw(_ptr(logits), n, _ptr(seen), ctypes.byref(params), _ptr(best), _ptr(workspace),
                                workspace_bytes, _stream(stream)), "sample_draw")


def sample_mark(tok, seen, n: int, stream=None) -> None:
    """src/lfm/sample.rs:332 encode_mark: the drawn token into the seen bitmap."""
    check(load().mh_sample_mark(_ptr(tok), _ptr(seen), n, _stream(stream)), "sample_mark")


class TensorMeta(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("ndim", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 8),
                ("bytes", ctypes.c_uint64)]


class Checkpoint:
    """src/safetensors.rs Checkpoint over the C ABI: names, metadata, staged reads to device memory."""

    def __init__(self, directory: str):
        h = _vp()
        check(load().mh_checkpoint_open(os.fsencode(directory), ctypes.byref(h)), "checkpoint_open")
        self._h = h

    def close(self) -> None:
        if self._h:
            load().mh_checkpoint_close(self._h)
            self._h = _vp()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def names(self) -> list[str]:
        lib = load()
        return [lib.mh_checkpoint_name(self._h, i).decode() for i in range(lib.mh_checkpoint_count(self._h))]

    def meta(self, name: str):
        """(dtype, shape, bytes) with dtype one of MH_DTYPE_*."""
        m = TensorMeta()
        check(load().mh_checkpoint_meta(self._h, name.encode(), ctypes.byref(m)), "checkpoint_meta")
        return m.dtype, tuple(m.shape[i] for i in range(m.ndim)), m.bytes

    def read(self, name: str, dst, nbytes: int, stream=None) -> None:
        check(load().mh_checkpoint_read(self._h, name.encode(), _ptr(dst), nbytes, _stream(stream)),
              "checkpoint_read")

    def load_quant(self, base: str, rows: int, k: int, bits: int, codes, scales, biases,
                   stream=None) -> "QuantWeights":
        out = CQuantWeights()
        check(load().mh_load_quant(self._h, base.encode(), rows, k, bits, _ptr(codes), _ptr(scales),
                                   _ptr(biases), ctypes.byref(out), _stream(stream)), "load_quant")
        return QuantWeights(codes, scales, biases, rows, k, 64, bits)


def gemv_gather_act(gate: QuantWeights, up: QuantWeights, x, ids, act, topk: int, n_inter: int,
                    stream=None) -> None:
    """src/kernels/lfm.rs:421."""
    check(load().mh_gemv_gather_act(_qref(gate), _qref(up), _ptr(x), _ptr(ids), _ptr(act), topk,
                                    n_inter, _stream(stream)), "gemv_gather_act")


def gemv_gu_act(gate: QuantWeights, up: QuantWeights, x, act, stream=None) -> None:
    """src/kernels/lfm.rs:464."""
    check(load().mh_gemv_gu_act(_qref(gate), _qref(up), _ptr(x), _ptr(act), _stream(stream)),
          "gemv_gu_act")


def gemv_gather_down_combine4(down: QuantWeights, act, ids, weights, out, topk: int = 4,
                              n_out: int = 2048, stream=None) -> None:
    """src/kernels/lfm.rs:499 (topk 1..4 here)."""
    check(load().mh_gemv_gather_down_combine(_qref(down), _ptr(act), _ptr(ids), _ptr(weights),
                                             _ptr(out), topk, n_out, _stream(stream)),
          "gemv_gather_down_combine4")


def moe_decode(router, bias, gate: QuantWeights, up: QuantWeights, down: QuantWeights,
               n_experts: int, topk: int, x, out, logits, ids, weights, act, scratch,
               mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """One MoE decode step (src/lfm.rs:967-1011).  scratch: MOE_DECODE_SCRATCH_WORDS
    u32 words, zeroed once before the first call, then left to this function."""
    check(load().mh_moe_decode(_ptr(router), _dtype_of(router), _ptr(bias), mode, eps,
                               _qref(gate), _qref(up), _qref(down), n_experts, topk, _ptr(x),
                               _ptr(out), _ptr(logits), _ptr(ids), _ptr(weights), _ptr(act),
                               _ptr(scratch), _stream(stream)), "moe_decode")


MOE_DECODE_STAMPS = 10  # MH_MOE_DECODE_STAMPS
MOE_DECODE_STAMP_WAVES = 2048  # MH_MOE_DECODE_STAMP_WAVES


def moe_decode_stamped(router, bias, gate: QuantWeights, up: QuantWeights, down: QuantWeights,
                       n_experts: int, topk: int, x, out, logits, ids, weights, act, scratch, stamps,
                       mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """moe_decode on the single-launch path with per-wave phase timestamps
    (measurement only): stamps u64 [MOE_DECODE_STAMP_WAVES * MOE_DECODE_STAMPS]."""
    check(load().mh_moe_decode_stamped(_ptr(router), _dtype_of(router), _ptr(bias), mode, eps,
                                       _qref(gate), _qref(up), _qref(down), n_experts, topk, _ptr(x),
                                       _ptr(out), _ptr(logits), _ptr(ids), _ptr(weights), _ptr(act),
                                       _ptr(scratch), _ptr(stamps), _stream(stream)), "moe_decode_stamped")


def router_prefill(x, w, out, m: int, k: int, e: int, stream=None) -> None:
    """src/kernels/lfm.rs:366."""
    check(load().mh_router_prefill(_ptr(x), _ptr(w), _dtype_of(w), _ptr(out), m, k, e,
                                   _stream(stream)), "router_prefill")


def moe_route_batch(logits, bias, ids, gw, m: int, e: int, topk: int,
                    mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """src/kernels/lfm.rs:536."""
    check(load().mh_moe_route_batch(_ptr(logits), _ptr(bias), _ptr(ids), _ptr(gw), m, e, topk,
                                    mode, eps, _stream(stream)), "moe_route_batch")


# ------------------------------------------------------- prefill MoE ops --

class MoeTile:
    """Row x column tile of a grouped GEMM block map (src/kernels/quant.rs:19-40).
    T32 / T128 are the reference's shapes; GU128 / DN128 are MI355X tiles of
    128 rows; GU512 / DN512 map whole expert segments of up to 512 rows (the
    segment kernels the fused prefill uses for gate/up and down)."""

    T32 = (32, 64)
    T128 = (128, 64)
    GU128 = (128, 128)
    DN128 = (128, 256)
    GU512 = (512, 128)
    DN512 = (512, 256)


def moe_zero_counts(counts, e: int, stream=None) -> None:
    check(load().mh_moe_zero_counts(_ptr(counts), e, _stream(stream)), "moe_zero_counts")


def moe_count_slots(ids, counts, s: int, e: int, stream=None) -> None:
    check(load().mh_moe_count_slots(_ptr(ids), _ptr(counts), s, e, _stream(stream)),
          "moe_count_slots")


def moe_offsets(counts, offsets, e: int, stream=None) -> None:
    check(load().mh_moe_offsets(_ptr(counts), _ptr(offsets), e, _stream(stream)), "moe_offsets")


def moe_sorted(ids, offsets, ids_sorted, slotpos, m: int, e: int, topk: int, stream=None) -> None:
    check(load().mh_moe_sorted(_ptr(ids), _ptr(offsets), _ptr(ids_sorted), _ptr(slotpos), m, e,
                               topk, _stream(stream)), "moe_sorted")


def moe_zero_blocks(gu, dn, n_gu: int, n_dn: int, stream=None) -> None:
    check(load().mh_moe_zero_blocks(_ptr(gu), _ptr(dn), n_gu, n_dn, _stream(stream)),
          "moe_zero_blocks")


def moe_block_offsets(counts, gu_off, dn_off, e: int, bm: int, gu_bn: int, dn_bn: int,
                      gu_n: int, dn_n: int, stream=None) -> None:
    check(load().mh_moe_block_offsets(_ptr(counts), _ptr(gu_off), _ptr(dn_off), e, bm, gu_bn,
                                      dn_bn, gu_n, dn_n, _stream(stream)), "moe_block_offsets")


def moe_blocks(counts, offsets, gu_off, dn_off, gu, max_gu: int, dn, max_dn: int, e: int, bm: int,
               gu_bn: int, dn_bn: int, gu_n: int, dn_n: int, stream=None) -> None:
    check(load().mh_moe_blocks(_ptr(counts), _ptr(offsets), _ptr(gu_off), _ptr(dn_off), _ptr(gu),
                               max_gu, _ptr(dn), max_dn, e, bm, gu_bn, dn_bn, gu_n, dn_n,
                               _stream(stream)), "moe_blocks")


def gather_rows_bf16(table, ids, out, m: int, h: int, n_table: int, stream=None) -> None:
    """src/kernels/elementwise.rs:59."""
    check(load().mh_gather_rows_bf16(_ptr(table), _ptr(ids), _ptr(out), m, h, n_table,
                                     _stream(stream)), "gather_rows_bf16")


def silu_mul_bf16(gate, up, out, n: int, stream=None) -> None:
    """src/kernels/elementwise.rs:48."""
    check(load().mh_silu_mul_bf16(_ptr(gate), _ptr(up), _ptr(out), n, _stream(stream)),
          "silu_mul_bf16")


def moe_combine_rows(sorted_rows, slotpos, weights, out, m: int, h: int, topk: int,
                     stream=None) -> None:
    """src/kernels/lfm.rs:701."""
    check(load().mh_moe_combine_rows(_ptr(sorted_rows), _ptr(slotpos), _ptr(weights), _ptr(out), m,
                                     h, topk, _stream(stream)), "moe_combine_rows")


def gemm_q4_grouped_mlx(a, w: QuantWeights, c, blocks, n_blocks: int, s_rows: int, n: int,
                        tile=MoeTile.T128, stream=None) -> None:
    """src/kernels/quant.rs:223."""
    check(load().mh_gemm_q4_grouped(_ptr(a), _qref(w), _ptr(c), _ptr(blocks), n_blocks, s_rows, n,
                                    tile[0], tile[1], _stream(stream)), "gemm_q4_grouped_mlx")


def gemm_q4_grouped_mlx_gu(a, gate: QuantWeights, up: QuantWeights, gate_out, up_out, blocks,
                           n_blocks: int, s_rows: int, n: int, tile=MoeTile.T32,
                           stream=None) -> None:
    """src/kernels/quant.rs:151."""
    check(load().mh_gemm_q4_grouped_gu(_ptr(a), _qref(gate), _qref(up), _ptr(gate_out),
                                       _ptr(up_out), _ptr(blocks), n_blocks, s_rows, n, tile[0],
                                       tile[1], _stream(stream)), "gemm_q4_grouped_mlx_gu")


def gemm_q4_grouped_gu_act(x, ids_sorted, x_rows: int, gate: QuantWeights, up: QuantWeights, act,
                           blocks, n_blocks: int, s_rows: int, n: int, tile=MoeTile.GU128,
                           stream=None) -> None:
    """gate/up + SwiGLU with the row gather fused (no reference counterpart)."""
    check(load().mh_gemm_q4_grouped_gu_act(_ptr(x), _ptr(ids_sorted), x_rows, _qref(gate),
                                           _qref(up), _ptr(act), _ptr(blocks), n_blocks, s_rows,
                                           n, tile[0], tile[1], _stream(stream)),
          "gemm_q4_grouped_gu_act")


def map_grid(n_entries: int, nt: int) -> int:
    """Workgroups of a grouped-GEMM launch over n_entries map entries of nt
    column tiles each: whole units of 8 x nt (the entries of a launch-ordered
    map)."""
    unit = 8 * nt
    return -(-n_entries // unit) * unit


def gemm_q4_grouped_ordered(a, w: QuantWeights, c, ord_map, n_entries: int, s_rows: int, n: int,
                            tile=MoeTile.DN512, stream=None) -> None:
    """The grouped GEMM over a launch-ordered block map (no reference
    counterpart): entry b is workgroup b's; n_entries = map_grid(...)."""
    check(load().mh_gemm_q4_grouped_ordered(_ptr(a), _qref(w), _ptr(c), _ptr(ord_map), n_entries, s_rows, n,
                                            tile[0], tile[1], _stream(stream)), "gemm_q4_grouped_ordered")


def gemm_q4_grouped_gu_act_ordered(x, ids_sorted, x_rows: int, gate: QuantWeights, up: QuantWeights, act,
                                   ord_map, n_entries: int, s_rows: int, n: int, tile=MoeTile.GU512,
                                   stream=None) -> None:
    """gate/up + SwiGLU with the row gather, over a launch-ordered block map
    (no reference counterpart)."""
    check(load().mh_gemm_q4_grouped_gu_act_ordered(_ptr(x), _ptr(ids_sorted), x_rows, _qref(gate), _qref(up),
                                                   _ptr(act), _ptr(ord_map), n_entries, s_rows, n, tile[0],
                                                   tile[1], _stream(stream)), "gemm_q4_grouped_gu_act_ordered")


PREFILL_WS_REGIONS = ["logits", "ids", "gw", "counts", "offsets", "ids_sorted", "slotpos",
                      "gu_off", "dn_off", "gu_map", "dn_map", "act", "ed", "gu_ord", "dn_ord"]


def moe_prefill_workspace(m: int, n_experts: int, topk: int, d_model: int, n_inter: int):
    """(total bytes, {region: byte offset}) of mh_moe_prefill's workspace."""
    offs = (ctypes.c_size_t * len(PREFILL_WS_REGIONS))()
    total = load().mh_moe_prefill_workspace(m, n_experts, topk, d_model, n_inter, offs)
    return int(total), dict(zip(PREFILL_WS_REGIONS, [int(o) for o in offs]))


def moe_prefill(router, bias, gate: QuantWeights, up: QuantWeights, down: QuantWeights,
                n_experts: int, topk: int, x, m: int, out, workspace, workspace_bytes: int,
                mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """src/lfm.rs:847-965 moe_prefill as one call."""
    check(load().mh_moe_prefill(_ptr(router), _dtype_of(router), _ptr(bias), mode, eps,
                                _qref(gate), _qref(up), _qref(down), n_experts, topk, _ptr(x), m,
                                _ptr(out), _ptr(workspace), workspace_bytes, _stream(stream)),
          "moe_prefill")


PREFILL_STAMP_WGS = 4096  # MH_PREFILL_STAMP_WGS
PREFILL_STAMPS = 4  # MH_PREFILL_STAMPS


def moe_prefill_stamped(router, bias, gate: QuantWeights, up: QuantWeights, down: QuantWeights,
                        n_experts: int, topk: int, x, m: int, out, workspace, workspace_bytes: int, stamps,
                        mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """moe_prefill with the grouped GEMMs' workgroups stamped (measurement
    only): stamps u64 [2 * PREFILL_STAMP_WGS * PREFILL_STAMPS]."""
    check(load().mh_moe_prefill_stamped(_ptr(router), _dtype_of(router), _ptr(bias), mode, eps,
                                        _qref(gate), _qref(up), _qref(down), n_experts, topk, _ptr(x), m,
                                        _ptr(out), _ptr(workspace), workspace_bytes, _ptr(stamps), _stream(stream)),
          "moe_prefill_stamped")
