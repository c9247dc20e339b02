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


def _bf16_ulp(v):
    """bf16 ulp at |v| (2^(e - 7)); the least normal's for zero and denormals."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def float_report(got_bf16, want, name=""):
    """Compares bf16 outputs (uint16 bit patterns) with a reference (float64
    values, or bf16 bit patterns): prints the literal max abs err, the
    rel-L2 error and a histogram of the error in bf16 ulps of the reference
    (0, 1, 2, 3-8, > 8), and returns (max_abs, rel_l2, max|ref|)."""
    from molten_amd import layout

    g = layout.bf16_to_f32(np.asarray(got_bf16, np.uint16)).astype(np.float64)
    w = np.asarray(want)
    w = layout.bf16_to_f32(w).astype(np.float64) if w.dtype == np.uint16 else w.astype(np.float64)
    assert np.isfinite(g).all(), f"{name}: non-finite outputs"
    d = np.abs(g - w)
    max_abs = float(d.max()) if d.size else 0.0
    rel_l2 = float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30))
    ulps = d / _bf16_ulp(w)
    hist = [int((ulps == 0).sum()), int(((ulps > 0) & (ulps <= 1)).sum()), int(((ulps > 1) & (ulps <= 2)).sum()),
            int(((ulps > 2) & (ulps <= 8)).sum()), int((ulps > 8).sum())]
    print(f"{name}: max abs err {max_abs:.4g} (max |ref| {np.abs(w).max():.4g}), rel-L2 {rel_l2:.3g}, "
          f"bf16-ulp histogram [0, <=1, <=2, <=8, >8] = {hist}", flush=True)
    return max_abs, rel_l2, float(np.abs(w).max())


def assert_tolerance(got_bf16, want, name="", rel_l2_max=5e-3, abs_frac=2e-2):
    """The stated float tolerance: rel-L2 <= 5e-3 and max abs err <= 2e-2 x
    max |ref| (bf16 outputs of magnitude ~1e3 carry 4-8 per ulp, so the
    absolute bound is taken relative to the output scale); the literal max
    abs err is printed beside it."""
    max_abs, rel_l2, scale = float_report(got_bf16, want, name)
    assert rel_l2 <= rel_l2_max, (name, rel_l2)
    assert max_abs <= abs_frac * max(scale, 1.0), (name, max_abs, scale)
