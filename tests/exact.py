"""Exact rational helpers for pinning the oracle (independent of oracle/ks_oracle.c).

Values are fractions.Fraction; rounding to a binary format is done from first
principles (significand width, minimum exponent, ties-to-even), so a mistake in
the C oracle's integer rounding would not be mirrored here.
"""
from fractions import Fraction
import math
import struct


def bf16_value(bits: int) -> Fraction:
    f = struct.unpack("<f", struct.pack("<I", (bits & 0xFFFF) << 16))[0]
    return Fraction(f)


def f32_value(x: float) -> Fraction:
    return Fraction(struct.unpack("<f", struct.pack("<f", x))[0])


def round_binary(v: Fraction, mant_bits: int, emin: int, emax: int) -> Fraction:
    """Round v to the nearest value with `mant_bits` significant bits (incl. the leading
    one), minimum normal exponent emin (subnormals below), ties to even. Overflow -> inf."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix floating error in log2
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    q = Fraction(2) ** (e - (mant_bits - 1))
    n = a / q
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * q
    if r >= Fraction(2) ** (emax + 1):
        return sign * Fraction(10) ** 400  # stands for infinity
    return sign * r


def round_bf16(v: Fraction) -> Fraction:
    return round_binary(v, 8, -126, 127)


def round_f32(v: Fraction) -> Fraction:
    return round_binary(v, 24, -126, 127)


def to_bf16_bits(v: Fraction) -> int:
    """bits of an exactly representable bf16 value (0 -> +0)."""
    f = float(v)
    u = struct.unpack("<I", struct.pack("<f", f))[0]
    assert u & 0xFFFF == 0, "value not representable in bf16"
    return u >> 16


def to_f32(v: Fraction) -> float:
    return struct.unpack("<f", struct.pack("<f", float(v)))[0]
