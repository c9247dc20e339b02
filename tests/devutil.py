"""Test helpers: move numpy arrays (bf16 as uint16, u32) to and from the GPU
as torch tensors with the same bytes.  torch is only the allocator here."""
import numpy as np
import torch

from molten_amd import hip

_VIEW = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32,
         np.dtype(np.uint64): np.int64, np.dtype(np.uint8): np.uint8}


def to_dev(a: np.ndarray, device="cuda:0") -> torch.Tensor:
    a = np.ascontiguousarray(a)
    v = a.view(_VIEW.get(a.dtype, a.dtype))
    return torch.from_numpy(v.copy()).to(device)


def from_dev(t: torch.Tensor, dtype) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy().view(dtype)


def empty_dev(shape, dtype, device="cuda:0") -> torch.Tensor:
    tdt = {np.uint16: torch.int16, np.uint32: torch.int32, np.uint64: torch.int64,
           np.float32: torch.float32, np.uint8: torch.uint8}[dtype]
    return torch.empty(shape, dtype=tdt, device=device)


def zeros_dev(shape, dtype, device="cuda:0") -> torch.Tensor:
    t = empty_dev(shape, dtype, device)
    t.zero_()
    return t


def dev_quant(h, device="cuda:0"):
    """Upload a HostQuant; returns (hip.QuantWeights, keepalive tensors)."""
    c, s, b = to_dev(h.codes, device), to_dev(h.scales, device), to_dev(h.biases, device)
    return hip.QuantWeights(c, s, b, h.n, h.k, h.group_size, h.bits), (c, s, b)
