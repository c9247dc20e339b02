"""MLX affine weight layout and synthetic inputs (numpy only).

The on-disk / in-HBM format molten loads unchanged (src/weights.rs:11-30,
src/lfm.rs:283-316): codes U32 [out, in*bits/32] with code j of a row at bit
bits*j of the row's little-endian byte stream (Q4: eight codes per word, low
nibble first, lfm.metal:102-109; Q6: four codes per three bytes,
lfm.metal:186-199), and bf16 scale / bias per group of `group_size` inputs,
w = scale * q + bias.

bf16 tensors are carried as uint16 bit patterns.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def f32_to_bf16(a) -> np.ndarray:
    """Round float32 to bfloat16 bit patterns, nearest-even; NaN -> quiet NaN."""
    u = np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + (0x7FFF + ((u >> 16) & 1))).astype(np.uint32) >> 16
    r = np.where(nan, (u >> 16) | 0x0040, r)
    return r.astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_codes(q: np.ndarray, bits: int) -> np.ndarray:
    """Pack codes [rows, k] (values < 2**bits) into U32 [rows, k*bits/32]."""
    q = np.asarray(q, dtype=np.uint64)
    rows, k = q.shape
    if (k * bits) % 32:
        raise ValueError(f"k={k} at {bits} bits does not fill whole words")
    if bits == 4:
        q = q.reshape(rows, k // 8, 8)
        shifts = (4 * np.arange(8, dtype=np.uint64))[None, None, :]
        return (q << shifts).sum(axis=2).astype(np.uint32)
    if bits == 6:
        # four codes -> 24 bits -> three bytes
        q = q.reshape(rows, k // 4, 4)
        v = (q << (6 * np.arange(4, dtype=np.uint64))[None, None, :]).sum(axis=2)
        b = np.stack([(v >> s) & 0xFF for s in (0, 8, 16)], axis=2).astype(np.uint8)
        return b.reshape(rows, -1).view(np.uint32).reshape(rows, k * 6 // 32)
    if bits == 8:
        return q.astype(np.uint8).reshape(rows, k).view(np.uint32).reshape(rows, k // 4)
    raise ValueError(f"unsupported bits {bits}")


def unpack_codes(codes: np.ndarray, bits: int, k: int) -> np.ndarray:
    """Inverse of pack_codes: U32 [rows, k*bits/32] -> uint8 [rows, k]."""
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    rows = codes.shape[0]
    if bits == 4:
        shifts = (4 * np.arange(8, dtype=np.uint32))[None, None, :]
        return ((codes[:, :, None] >> shifts) & 0xF).reshape(rows, k).astype(np.uint8)
    if bits == 6:
        b = codes.view(np.uint8).reshape(rows, k // 4, 3).astype(np.uint32)
        v = b[:, :, 0] | (b[:, :, 1] << 8) | (b[:, :, 2] << 16)
        return np.stack([(v >> (6 * i)) & 63 for i in range(4)], axis=2).reshape(rows, k).astype(
            np.uint8
        )
    if bits == 8:
        return codes.view(np.uint8).reshape(rows, k).copy()
    raise ValueError(f"unsupported bits {bits}")


@dataclass
class HostQuant:
    """Host copy of one MLX affine matrix (numpy)."""

    codes: np.ndarray  # uint32 [n, k*bits/32]
    scales: np.ndarray  # uint16 (bf16) [n, k/gs]
    biases: np.ndarray  # uint16 (bf16) [n, k/gs]
    n: int
    k: int
    group_size: int
    bits: int

    def dequant_f64(self) -> np.ndarray:
        """W[n, k] = s*q + b in float64 (no rounding): the semantic matrix."""
        q = unpack_codes(self.codes, self.bits, self.k).astype(np.float64)
        s = np.repeat(bf16_to_f32(self.scales).astype(np.float64), self.group_size, axis=1)
        b = np.repeat(bf16_to_f32(self.biases).astype(np.float64), self.group_size, axis=1)
        return s * q + b


def synth_quant(rng: np.random.Generator, n: int, k: int, bits: int, group_size: int = 64,
                scale_std: float = 0.02, bias_std: float = 0.02) -> HostQuant:
    """BASELINE's synthetic weights: uniform codes, s = |N(0, .02)| + 1e-3,
    b = N(0, .02), both rounded to bf16."""
    words = k * bits // 32
    codes = rng.integers(0, 2**32, size=(n, words), dtype=np.uint64).astype(np.uint32)
    g = k // group_size
    scales = f32_to_bf16(np.abs(rng.normal(0.0, scale_std, size=(n, g))) + 1e-3)
    biases = f32_to_bf16(rng.normal(0.0, bias_std, size=(n, g)))
    return HostQuant(codes, scales, biases, n, k, group_size, bits)


def synth_bf16(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return f32_to_bf16(rng.normal(0.0, std, size=shape))
