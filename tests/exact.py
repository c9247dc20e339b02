"""Exact f32 arithmetic for tests: a fused multiply-add computed with
rationals and rounded once to the nearest f32 (ties to even), independent of
any C library.  Used to replay the chunk order on tiny shapes and pin the
oracle bit for bit."""
from __future__ import annotations

from fractions import Fraction

import numpy as np

_TWO = Fraction(2)


def _round_f32(q: Fraction) -> np.float32:
    if q == 0:
        return np.float32(0.0)
    sign = -1.0 if q < 0 else 1.0
    a = -q if q < 0 else q
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if _TWO**e > a:
        e -= 1
    elif _TWO ** (e + 1) <= a:
        e += 1
    qexp = max(e - 23, -149)
    scaled = a / _TWO**qexp
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = Fraction(n) * _TWO**qexp
    if val >= _TWO**128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(val))


def _neg_zero(v: np.float32) -> bool:
    return v == 0 and np.signbit(v)


def fma32(a, b, c) -> np.float32:
    """round_f32(a*b + c) exactly (IEEE fusedMultiplyAdd, round to nearest even)."""
    a, b, c = np.float32(a), np.float32(b), np.float32(c)
    if not (np.isfinite(a) and np.isfinite(b) and np.isfinite(c)):
        return np.float32(np.float64(a) * np.float64(b) + np.float64(c))
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if exact == 0:
        prod_neg = (np.signbit(a) != np.signbit(b))
        prod_zero = (a == 0 or b == 0)
        if prod_zero and c == 0 and prod_neg and np.signbit(c):
            return np.float32(-0.0)
        return np.float32(0.0)
    return _round_f32(exact)


def add32(a, b) -> np.float32:
    return np.float32(np.float32(a) + np.float32(b))


def mul32(a, b) -> np.float32:
    return np.float32(np.float32(a) * np.float32(b))


def butterfly64(a):
    a = [np.float32(v) for v in a]
    m = 1
    while m < 64:
        a = [add32(a[l], a[l ^ m]) for l in range(64)]
        m <<= 1
    return a[0]


def replay_qrow(q, xf, s, b, gs):
    """Chunk-order value of one quantized row.
    q: codes [k] ints; xf: f32 x [k]; s, b: f32 per group."""
    k = len(q)
    C = k // 32
    lanes = [np.float32(0.0)] * 64
    for c in range(C):
        p = np.float32(0.0)
        xs = np.float32(0.0)
        for i in range(32):
            kk = 32 * c + i
            p = fma32(np.float32(q[kk]), xf[kk], p)
            xs = add32(xs, xf[kk])
        g = (32 * c) // gs
        h = fma32(s[g], p, mul32(b[g], xs))
        lanes[c % 64] = add32(lanes[c % 64], h)
    return butterfly64(lanes)


def replay_dense_row(w, xf):
    k = len(w)
    lanes = [np.float32(0.0)] * 64
    for c in range(k // 32):
        p = np.float32(0.0)
        for i in range(32):
            p = fma32(w[32 * c + i], xf[32 * c + i], p)
        lanes[c % 64] = add32(lanes[c % 64], p)
    return butterfly64(lanes)
