"""Exact-arithmetic helpers for the tests: float32 rounding of exact
rationals, so that a fused multiply-add and an integer-to-float conversion
can be evaluated independently of any hardware FMA."""
from fractions import Fraction

import numpy as np


def round_f32(v, neg_zero=False):
    """The float32 nearest to the rational v, ties to even (overflow to inf)."""
    if v == 0:
        return np.float32(-0.0) if neg_zero else np.float32(0.0)
    sign = -1 if v < 0 else 1
    a = abs(Fraction(v))
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    shift = max(e, -126) - 23
    q = a / Fraction(2) ** shift
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    res = Fraction(n) * Fraction(2) ** shift
    if res >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(res))


def fma32(a, b, c):
    """a*b + c rounded once to float32 (a, b, c float32)."""
    a, b, c = np.float32(a), np.float32(b), np.float32(c)
    p = Fraction(float(a)) * Fraction(float(b))
    s = p + Fraction(float(c))
    if s == 0:
        # IEEE: an exact zero sum is +0 unless both terms are -0
        neg = (p == 0 and np.signbit(a) != np.signbit(b)) and (c == 0 and np.signbit(c))
        return round_f32(0, neg)
    return round_f32(s)


def mul32(a, b):
    return round_f32(Fraction(float(np.float32(a))) * Fraction(float(np.float32(b))))


def i2f32(i):
    """int32 to float32, round to nearest even."""
    return round_f32(Fraction(int(i)))
