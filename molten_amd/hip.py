"""ctypes binding of libmolten_hip.so: the operator layer of molten's hot path.

Each function mirrors one operator wrapper of the reference's Rust layer
(src/kernels/lfm.rs, src/kernels/quant.rs, src/kernels/elementwise.rs): same
name, same argument order and meaning, and it raises `MoltenError` where the
reference's `ensure!` would return an error.  Tensors are torch tensors on
the GPU (only their device pointers cross the C ABI) or plain integer device
addresses.  This is the Python counterpart of the Rust `src/hip.rs` binding
shown in INTEGRATION.md.

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
    "mh_dequant_to_bf16": [_qw, _vp, _vp],
    "mh_dequant_q4_bf16_bulk": [_qw, _vp, _vp],
    "mh_gemv_quant": [_qw, _vp, _vp, _u32, _vp],
    "mh_gemv_head_argmax": [_qw, _vp, _vp, _u32, _vp],
    "mh_gemv_quant_argmax": [_qw, _vp, _vp, _vp, _vp, _vp, _u32, _vp],
    "mh_token_tail": [_vp, _vp, _u32, _vp],
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
    "mh_router_prefill": [_vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp],
    "mh_moe_route_batch": [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _i32, _f32, _vp],
}
_RESTYPES = {"mh_last_error": ctypes.c_char_p, "mh_version": ctypes.c_char_p}

_lib: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the native library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(path)
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
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

def gemv_quant(w: QuantWeights, x, y, batch: int = 1, stream=None) -> None:
    """src/kernels/lfm.rs:112 (batch > 1 is this build's extension)."""
    check(load().mh_gemv_quant(_qref(w), _ptr(x), _ptr(y), batch, _stream(stream)), "gemv_quant")


def gemv_head_argmax(w: QuantWeights, x, best, batch: int = 1, stream=None) -> None:
    """src/kernels/lfm.rs:826."""
    check(load().mh_gemv_head_argmax(_qref(w), _ptr(x), _ptr(best), batch, _stream(stream)),
          "gemv_head_argmax")


def gemv_quant_argmax(w: QuantWeights, x, y, best, done=None, ids=None, batch: int = 1,
                      stream=None) -> None:
    """Stored logits + argmax (BASELINE configs 2 and 5)."""
    check(load().mh_gemv_quant_argmax(_qref(w), _ptr(x), _ptr(y), _ptr(best), _ptr(done),
                                      _ptr(ids), batch, _stream(stream)), "gemv_quant_argmax")


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
               n_experts: int, topk: int, x, out, logits, ids, weights, act, counter,
               mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """One MoE decode step (src/lfm.rs:967-1011)."""
    check(load().mh_moe_decode(_ptr(router), _dtype_of(router), _ptr(bias), mode, eps,
                               _qref(gate), _qref(up), _qref(down), n_experts, topk, _ptr(x),
                               _ptr(out), _ptr(logits), _ptr(ids), _ptr(weights), _ptr(act),
                               _ptr(counter), _stream(stream)), "moe_decode")


def router_prefill(x, w, out, m: int, k: int, e: int, stream=None) -> None:
    """src/kernels/lfm.rs:366."""
    check(load().mh_router_prefill(_ptr(x), _ptr(w), _dtype_of(w), _ptr(out), m, k, e,
                                   _stream(stream)), "router_prefill")


def moe_route_batch(logits, bias, ids, gw, m: int, e: int, topk: int,
                    mode: int = ROUTE_SIGMOID_BIAS, eps: float = 1e-6, stream=None) -> None:
    """src/kernels/lfm.rs:536."""
    check(load().mh_moe_route_batch(_ptr(logits), _ptr(bias), _ptr(ids), _ptr(gw), m, e, topk,
                                    mode, eps, _stream(stream)), "moe_route_batch")
