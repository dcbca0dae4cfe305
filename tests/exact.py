"""Exact-rational IEEE binary32 arithmetic for pinning the oracle: every operation is computed exactly with
Fractions and rounded once, to nearest even, to binary32 (subnormals and overflow included)."""
import math
from fractions import Fraction

import numpy as np

_MIN_EXP = -126          # smallest normal exponent
_MANT = 23
_MAX = Fraction(2) ** 128 - Fraction(2) ** 104          # largest finite binary32
_OVF = Fraction(2) ** 128 - Fraction(2) ** 103          # rounding threshold to infinity


def F(x):
    """Exact value of a float32 (or Python float already holding one); Fractions pass through."""
    if isinstance(x, Fraction):
        return x
    x = float(np.float32(x))
    if not math.isfinite(x):
        raise ValueError('non-finite')
    return Fraction(x)


def _rne_int(q):
    """Round a non-negative Fraction to the nearest integer, ties to even."""
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        return fl + 1
    return fl


def rne(q):
    """Fraction -> np.float32, one rounding to nearest even."""
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    a = -q if q < 0 else q
    if a >= _OVF:
        return np.float32(sign * np.inf)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, _MIN_EXP)
    quantum = Fraction(2) ** (e - _MANT)
    k = _rne_int(a / quantum)
    val = k * quantum
    if val > _MAX:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(val))


def mul(a, b):
    return rne(F(a) * F(b))


def add(a, b):
    return rne(F(a) + F(b))


def div(a, b):
    return rne(F(a) / F(b))


def fma(a, b, c):
    return rne(F(a) * F(b) + F(c))


def sqrt(a):
    """Correctly rounded binary32 square root of a float32 a >= 0."""
    q = F(a)
    if q < 0:
        raise ValueError('sqrt of a negative value')
    if q == 0:
        return np.float32(0.0)
    K = 200
    scaled = q * Fraction(2) ** (2 * K)
    num = scaled.numerator // scaled.denominator
    s = math.isqrt(num)
    if s * s == scaled:                  # exact square root
        return rne(Fraction(s, 2 ** K))
    # the root lies strictly inside (s, s+1) / 2^K: its midpoint rounds the same way (K >> 24)
    return rne(Fraction(2 * s + 1, 2 ** (K + 1)))


def adam_elem(g, p, m, v, *, lr, b1, b2, eps, bc1, bc2, wd, mode, factor=None):
    """Appendix-B element sequence, one rounding per operation (all inputs float32 values)."""
    if factor is not None:
        g = mul(g, factor)
    if mode == 0:
        g = fma(wd, p, g)
    omb1 = rne(1 - F(b1))
    omb2 = rne(1 - F(b2))
    m2 = fma(b1, m, mul(omb1, g))
    v2 = fma(b2, v, mul(mul(omb2, g), g))
    mh = div(m2, bc1)
    vh = div(v2, bc2)
    den = add(sqrt(vh), eps)
    upd = div(mh, den)
    if mode == 1:
        upd = fma(wd, p, upd)
    p2 = fma(-F(lr), upd, p)
    return p2, m2, v2
