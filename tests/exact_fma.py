"""Exact-rational IEEE-754 binary32 fused multiply-add, for pinning the oracle.

Independent of any C library: every value is computed exactly with
fractions.Fraction and rounded once to the nearest binary32 (ties to even),
with gradual underflow and overflow to infinity, which is the definition of
fusedMultiplyAdd in IEEE 754-2008 section 5.4.1.  The signed-zero rules are the
standard's (6.3): an exact zero sum of non-zero operands is +0 in
round-to-nearest; a sum of two zeros is -0 only when both are -0; a non-zero
result that rounds to zero keeps its sign.

Only for small cases: a length-K chain costs K Fraction operations.
"""
from __future__ import annotations

import math
import struct
from fractions import Fraction

INF = float("inf")
NAN = float("nan")


def f32_from_bits(u: int) -> float:
    return struct.unpack("<f", struct.pack("<I", u & 0xFFFFFFFF))[0]


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def bf16_to_f32(h: int) -> float:
    """Exact widen (compiler/src/jit.rs:29225-29227), as arithmetic on bits."""
    return f32_from_bits((h & 0xFFFF) << 16)


def _pow2(e: int) -> Fraction:
    return Fraction(2) ** e if e >= 0 else Fraction(1, 2 ** (-e))


def round_f32(q: Fraction, neg_zero: bool = False) -> float:
    """Round the exact rational q to binary32, nearest-even.  `neg_zero`
    gives the sign when q == 0."""
    if q == 0:
        return -0.0 if neg_zero else 0.0
    sign = -1.0 if q < 0 else 1.0
    a = -q if q < 0 else q
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if _pow2(e) > a:
        e -= 1
    assert _pow2(e) <= a < _pow2(e + 1)
    if e > 127:
        return sign * INF
    qe = (e - 23) if e >= -126 else -149  # exponent of the last significand bit
    scaled = a / _pow2(qe)
    n = scaled.numerator // scaled.denominator
    r = scaled - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    if n == 0:
        return math.copysign(0.0, sign)
    val = Fraction(n) * _pow2(qe)
    if val >= _pow2(128):
        return sign * INF
    return sign * float(val)  # exact: a binary32 value is a binary64 value


def fma(a: float, b: float, c: float) -> float:
    """binary32 fusedMultiplyAdd(a, b, c); inputs must be binary32 values."""
    if math.isnan(a) or math.isnan(b) or math.isnan(c):
        return NAN
    if (math.isinf(a) and b == 0) or (math.isinf(b) and a == 0):
        return NAN
    psign = math.copysign(1.0, a) * math.copysign(1.0, b)
    if math.isinf(a) or math.isinf(b):
        if math.isinf(c) and math.copysign(1.0, c) != psign:
            return NAN
        return psign * INF
    if math.isinf(c):
        return c
    p = Fraction(a) * Fraction(b)
    if p == 0 and c == 0:
        return -0.0 if (psign < 0 and math.copysign(1.0, c) < 0) else 0.0
    s = p + Fraction(c)
    if s == 0:  # exact cancellation of non-zero terms
        return 0.0
    return round_f32(s)


def chain(xs, ws, init: float = 0.0) -> float:
    """The reference's per-element chain: acc = +0; acc = fma(x_k, w_k, acc)."""
    acc = init
    for x, w in zip(xs, ws):
        acc = fma(x, w, acc)
    return acc


def gemv(x_rows, w_logical_bits):
    """out[m][n] = chain over k of (x[m][k], bf16(w[n][k])) -- exact reference."""
    wf = [[bf16_to_f32(h) for h in row] for row in w_logical_bits]
    return [[chain(xr, wr) for wr in wf] for xr in x_rows]
