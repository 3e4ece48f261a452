"""Exact IEEE-754 binary arithmetic over ``fractions.Fraction``.

Every value is a ``Fraction``; ``round_binary`` rounds an exact rational to
the nearest value of a binary format with round-to-nearest, ties-to-even,
written from the definition of the format (no float hardware involved):

* a normal number ``|x|`` in ``[2**e, 2**(e+1))`` has the spacing
  ``2**(e - p + 1)`` (``p`` significand bits including the hidden one);
* below ``2**emin`` the spacing stays ``2**(emin - p + 1)`` (subnormals);
* the result is the multiple of the spacing nearest to ``x``; on a tie the
  one whose multiple count is even;
* a result at or above ``2**(emax + 1)`` overflows to infinity (returned as
  ``None``; callers here never reach it).

fp32 is ``p = 24, emin = -126, emax = 127``; bf16 is ``p = 8`` with the same
exponent range.  The module evaluates the Reposition's rotation and the
plausible mis-statements of it (a delta-angle rotation, division of each
product, fused multiply-adds), each operation rounded exactly as its form
states, so known answers computed here pin the oracle's operation order.
Signed zeros are not modelled: callers reject cases with a zero anywhere.
"""

from fractions import Fraction

import numpy as np

F32 = (24, -126, 127)
BF16 = (8, -126, 127)


def _floor_log2(a):
    """Largest e with 2**e <= a, for a positive Fraction."""
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    return e


def round_binary(x, fmt):
    p, emin, emax = fmt
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = max(_floor_log2(a), emin)
    spacing = Fraction(2) ** (e - p + 1)
    q = a / spacing
    n = q.numerator // q.denominator
    rest = q - n
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and n % 2 == 1):
        n += 1
    r = n * spacing
    if r >= Fraction(2) ** (emax + 1):
        return None
    return sign * r


def f32(x):
    return round_binary(x, F32)


def f32_from_bits(bits):
    """uint32 bit pattern -> exact Fraction of the fp32 value it encodes."""
    v = np.array([bits], dtype=np.uint32).view(np.float32)[0]
    if not np.isfinite(v):
        raise ValueError("finite values only")
    return Fraction(float(v))


def bf16_from_bits(bits):
    return f32_from_bits(np.uint32(int(bits) << 16))


def bits_f32(x):
    """An exact fp32 value (Fraction) -> its uint32 bit pattern."""
    if f32(x) != x:
        raise ValueError(f"{x} is not an fp32 value")
    return int(np.array([float(x)], dtype=np.float32).view(np.uint32)[0])


def bits_bf16(x):
    """An exact bf16 value (Fraction) -> its uint16 bit pattern."""
    if round_binary(x, BF16) != x:
        raise ValueError(f"{x} is not a bf16 value")
    return bits_f32(x) >> 16


def to_bf16_bits(y):
    """Round an fp32 value to bf16 (RNE) and return the uint16 bits."""
    return bits_bf16(round_binary(y, BF16))


# The rotation of one pair (x1, x2) from the old position's (co, so) to the
# new position's (cn, sn).  Every helper returns the two fp32 results.


def two_step(x1, x2, co, so, cn, sn):
    """Inverse rotation by the old angle with one division by cos^2 + sin^2,
    then the forward rotation by the new angle; each operation rounded."""
    s = f32(f32(co * co) + f32(so * so))
    u1 = f32(f32(f32(x1 * co) + f32(x2 * so)) / s)
    u2 = f32(f32(f32(x2 * co) - f32(x1 * so)) / s)
    y1 = f32(f32(u1 * cn) - f32(u2 * sn))
    y2 = f32(f32(u2 * cn) + f32(u1 * sn))
    return y1, y2


def delta_angle(x1, x2, co, so, cn, sn):
    """One rotation by the angle difference (cos and sin of new - old formed
    first, normalised by cos^2 + sin^2 of the old angle)."""
    s = f32(f32(co * co) + f32(so * so))
    cd = f32(f32(f32(cn * co) + f32(sn * so)) / s)
    sd = f32(f32(f32(sn * co) - f32(cn * so)) / s)
    y1 = f32(f32(x1 * cd) - f32(x2 * sd))
    y2 = f32(f32(x2 * cd) + f32(x1 * sd))
    return y1, y2


def per_term_division(x1, x2, co, so, cn, sn):
    """The two-step rotation with each product divided before the sum."""
    s = f32(f32(co * co) + f32(so * so))
    u1 = f32(f32(f32(x1 * co) / s) + f32(f32(x2 * so) / s))
    u2 = f32(f32(f32(x2 * co) / s) - f32(f32(x1 * so) / s))
    y1 = f32(f32(u1 * cn) - f32(u2 * sn))
    y2 = f32(f32(u2 * cn) + f32(u1 * sn))
    return y1, y2


def fused(x1, x2, co, so, cn, sn):
    """The two-step rotation with every ``a*b +- c*d`` contracted into
    ``fma(a, b, +-(c*d))``: one rounding for the first product and the sum."""
    s = f32(co * co + f32(so * so))
    u1 = f32(f32(x1 * co + f32(x2 * so)) / s)
    u2 = f32(f32(x2 * co - f32(x1 * so)) / s)
    y1 = f32(u1 * cn - f32(u2 * sn))
    y2 = f32(u2 * cn + f32(u1 * sn))
    return y1, y2


FORMS = {"two_step": two_step, "delta_angle": delta_angle, "per_term_division": per_term_division,
         "fused": fused}


def rotate_bf16_bits(form, x1_bits, x2_bits, co_bits, so_bits, cn_bits, sn_bits):
    """bf16 inputs and fp32 table entries (bit patterns) -> the bf16 bits of
    (y1, y2) under ``form``; ``None`` when a zero appears anywhere."""
    args = [bf16_from_bits(x1_bits), bf16_from_bits(x2_bits)] + \
           [f32_from_bits(b) for b in (co_bits, so_bits, cn_bits, sn_bits)]
    if any(a == 0 for a in args):
        return None
    y1, y2 = FORMS[form](*args)
    if y1 is None or y2 is None or y1 == 0 or y2 == 0:
        return None
    return to_bf16_bits(y1), to_bf16_bits(y2)
