"""Exact-rational model of IEEE binary32 / binary16 rounding (test utility).

An independent route to the values the oracle must produce: every operation
is carried out exactly on ``fractions.Fraction`` and then rounded to the
target format by the definition of round-to-nearest-even, without going
through numpy or the C library.  Used to pin the oracle's operation order.
"""

from fractions import Fraction
import math


def _round_to_format(v: Fraction, mant_bits: int, emin: int, emax: int) -> Fraction:
    """Round ``v`` to a binary format with ``mant_bits`` significand bits
    (hidden bit included), minimum normal exponent ``emin`` and maximum
    exponent ``emax``.  Returns +-inf as float('inf') wrapped in Fraction is
    impossible, so overflow raises OverflowError."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix e so that 2^e <= a < 2^(e+1)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)  # subnormal range uses the minimum exponent
    ulp = Fraction(2) ** (e - (mant_bits - 1))
    t = a / ulp
    n = t.numerator // t.denominator
    rem = t - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    r = n * ulp
    if r >= Fraction(2) ** (emax + 1):
        raise OverflowError("rounds to infinity")
    return sign * r


def f32(v) -> Fraction:
    """Exact value of ``v`` rounded to binary32 (RNE)."""
    return _round_to_format(Fraction(v), 24, -126, 127)


def f16(v) -> Fraction:
    """Exact value of ``v`` rounded to binary16 (RNE)."""
    return _round_to_format(Fraction(v), 11, -14, 15)


def rha(v: Fraction) -> int:
    """Round half away from zero, exactly."""
    a = abs(v)
    n = math.floor(a + Fraction(1, 2))
    return n if v >= 0 else -n


def rne(v: Fraction) -> int:
    """Round half to even, exactly."""
    n = math.floor(v)
    rem = v - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n
