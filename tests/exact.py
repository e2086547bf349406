"""Exact (rational) restatement of fp32 arithmetic, for pinning the oracle.

Independent of both the C oracle and the HIP kernels: every fp32 operation
is computed exactly with fractions.Fraction and rounded once to the nearest
float32 (ties to even), as IEEE 754 specifies. Slow; tiny shapes only.

  fma(a, b, c)  = round(a*b + c)            -- llvm.fma / vector.fma
  mulf, addf    = round(a*b), round(x + y)  -- arith.mulf / arith.addf
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np

_F32_MAX_EXP = 128        # values >= 2**128 round to inf
_F32_MIN_QUANTUM = -149   # subnormal spacing 2**-149
_F32_MANT = 24


def round_f32(x: Fraction, zero_sign: float = 1.0) -> float:
    """Nearest float32 to the exact rational x (ties to even), as a Python
    float. zero_sign gives the sign of an exactly-zero result."""
    if x == 0:
        return math.copysign(0.0, zero_sign)
    sign = -1.0 if x < 0 else 1.0
    a = -x if x < 0 else x
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = max(e - (_F32_MANT - 1), _F32_MIN_QUANTUM)
    scaled = a / (Fraction(2) ** q)
    n = scaled.numerator // scaled.denominator
    r = scaled - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = Fraction(n) * Fraction(2) ** q
    if val >= Fraction(2) ** _F32_MAX_EXP:
        return sign * math.inf
    return sign * float(val)


def _zero_sign_sum(x: float, y: float) -> float:
    # exact zero sum: -0 only when both addends are -0 (round to nearest)
    return -1.0 if (math.copysign(1.0, x) < 0 and math.copysign(1.0, y) < 0) else 1.0


def f32_add(x: float, y: float) -> float:
    if math.isnan(x) or math.isnan(y) or math.isinf(x) or math.isinf(y):
        return float(np.float32(x) + np.float32(y))
    return round_f32(Fraction(x) + Fraction(y), _zero_sign_sum(x, y))


def f32_mul(x: float, y: float) -> float:
    if math.isnan(x) or math.isnan(y) or math.isinf(x) or math.isinf(y):
        return float(np.float32(x) * np.float32(y))
    return round_f32(Fraction(x) * Fraction(y), math.copysign(1.0, x) * math.copysign(1.0, y))


def f32_fma(a: float, b: float, c: float) -> float:
    if any(math.isnan(v) or math.isinf(v) for v in (a, b, c)):
        return float(np.float32(np.float64(a) * np.float64(b) + np.float64(c)))
    p_sign = math.copysign(1.0, a) * math.copysign(1.0, b)
    zs = -1.0 if (p_sign < 0 and math.copysign(1.0, c) < 0) else 1.0
    return round_f32(Fraction(a) * Fraction(b) + Fraction(c), zs)


def maximumf0(x: float) -> float:
    """arith.maximumf(x, +0.0): NaN propagates; max(-0, +0) = +0."""
    if math.isnan(x):
        return x
    return x if x > 0 else 0.0


def minimumf0(x: float) -> float:
    """arith.minimumf(x, +0.0): NaN propagates; min(-0, +0) = -0."""
    if math.isnan(x):
        return x
    if x < 0:
        return x
    if x == 0:
        return x
    return 0.0


def if_relu0(x: float) -> float:
    """If(v > 0.0, v, 0.0): cmpf ogt is false for NaN and for -0, so both
    give the constant +0."""
    return x if x > 0 else 0.0


def dense_f32_exact(X, W, b, act: str, alpha: float, fma_path: bool) -> np.ndarray:
    """Per element: +0, then an ascending-k chain of fma (fma_path) or of
    mulf-then-addf; then addf bias, then the activation."""
    X = np.asarray(X, dtype=np.float32)
    W = np.asarray(W, dtype=np.float32)
    M, K = X.shape
    N = W.shape[1]
    Y = np.empty((M, N), dtype=np.float32)
    alpha32 = float(np.float32(alpha))
    for m in range(M):
        xr = [float(v) for v in X[m]]
        for n in range(N):
            acc = 0.0
            for k in range(K):
                a, w = xr[k], float(W[k, n])
                acc = f32_fma(a, w, acc) if fma_path else f32_add(acc, f32_mul(a, w))
            y = acc
            if b is not None:
                y = f32_add(y, float(np.float32(b[n])))
            if act == "relu":
                y = maximumf0(y)
            elif act == "if_relu":
                y = if_relu0(y)
            elif act == "leaky":
                y = f32_add(maximumf0(y), f32_mul(minimumf0(y), alpha32))
            Y[m, n] = y
    return Y


def dense_i32_exact(X, W, b, act: str) -> np.ndarray:
    """Exact integer sums reduced modulo 2^32 to two's complement (any
    summation order gives this result)."""
    X = np.asarray(X, dtype=np.int64)
    W = np.asarray(W, dtype=np.int64)
    M, K = X.shape
    N = W.shape[1]
    Y = np.empty((M, N), dtype=np.int32)
    for m in range(M):
        for n in range(N):
            s = sum(int(X[m, k]) * int(W[k, n]) for k in range(K))
            if b is not None:
                s += int(b[n])
            s = ((s + 2**31) % 2**32) - 2**31
            if act == "relu":
                s = s if s > 0 else 0
            Y[m, n] = s
    return Y
