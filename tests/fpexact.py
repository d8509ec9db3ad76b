"""Exact float32 arithmetic from rationals, to pin the oracle's fused
multiply-add and epilogue against the mathematics rather than against libm:
each operation is computed exactly (Fraction) and rounded once to float32 in
the requested IEEE mode, with IEEE 754's signs of zero."""
from fractions import Fraction
import math

import numpy as np

NEAREST, UPWARD, DOWNWARD, TOWARDZERO = 0, 1, 2, 3


def _fr(x):
    return Fraction(float(np.float32(x)))


def _neg(x):
    return bool(np.signbit(np.float32(x)))


def round_f32(fr, mode=NEAREST):
    """The float32 that fr rounds to (fr != 0)."""
    neg = fr < 0
    a = -fr if neg else fr
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                        # subnormals: the smallest exponent's spacing
    ulp = Fraction(2) ** (e - 23)
    k = a / ulp
    lo = math.floor(k)
    rem = k - lo
    if mode == NEAREST:
        up = rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1)
    elif mode == TOWARDZERO:
        up = False
    elif mode == UPWARD:
        up = rem > 0 and not neg
    else:
        up = rem > 0 and neg
    v = (lo + (1 if up else 0)) * ulp
    if v >= Fraction(2) ** 128:
        away = mode == NEAREST or (mode == UPWARD and not neg) or (mode == DOWNWARD and neg)
        big = np.float32(np.inf) if away else np.finfo(np.float32).max
        return np.float32(-big if neg else big)
    r = np.float32(float(v))
    return np.float32(-r) if neg else r


def _sum(p, p_neg, c, c_neg, mode):
    ex = p + c
    if ex != 0:
        return round_f32(ex, mode)
    if p == 0 and c == 0 and p_neg == c_neg:
        return np.float32(-0.0 if p_neg else 0.0)
    return np.float32(-0.0 if mode == DOWNWARD else 0.0)


def fma(a, b, c, mode=NEAREST):
    return _sum(_fr(a) * _fr(b), _neg(a) != _neg(b), _fr(c), _neg(c), mode)


def add(a, b, mode=NEAREST):
    return _sum(_fr(a), _neg(a), _fr(b), _neg(b), mode)


def mul(a, b, mode=NEAREST):
    ex = _fr(a) * _fr(b)
    if ex == 0:
        return np.float32(-0.0 if _neg(a) != _neg(b) else 0.0)
    return round_f32(ex, mode)


def i2f(s, mode=NEAREST):
    return np.float32(0.0) if s == 0 else round_f32(Fraction(int(s)), mode)


def epilogue(sums, dvals, ws, bias=None, old=None, mode=NEAREST):
    """The reference's per-output arithmetic (backend/kernels.h:60-68):
    acc = fma((float)s_b, d_b, acc) over the blocks in order, v = acc * ws,
    v = v + bias, out = old + v."""
    acc = np.float32(0.0)
    for s, d in zip(sums, dvals):
        acc = fma(i2f(s, mode), d, acc, mode)
    v = mul(acc, ws, mode)
    if bias is not None:
        v = add(v, bias, mode)
    if old is not None:
        v = add(old, v, mode)
    return v
