"""Pins oracle.reposition with closed forms a plausible mistake cannot pass.

Exact tables (cos/sin in {-m, 0, m}, m a power of two) make every rotation
exact, so a swapped sign, a cos/sin half swap, a wrong pair index, a dropped
division by cos^2 + sin^2 or a transposed operand gives a different answer.
"""

from fractions import Fraction

import numpy as np
import pytest

import exact_fp as ex
from oracle import bf16
from oracle import reposition as rp
from reposition_kat import KAT, KAT_VARIANTS, kat_expected, kat_pool


def _pool(rng, slots=8, heads=2, dim=8, layers=2, dtype="bf16"):
    k, v = [], []
    for _ in range(layers):
        kx = rng.standard_normal((slots, heads, dim)).astype(np.float32)
        vx = rng.standard_normal((slots, heads, dim)).astype(np.float32)
        k.append(bf16.from_f32(kx, dtype).reshape(kx.shape))
        v.append(bf16.from_f32(vx, dtype).reshape(vx.shape))
    return k, v


def _exact_table(rotary_dim, m=1.0):
    """Rows: 0 -> angle 0, 1 -> 90 degrees, 2 -> 180 degrees, scaled by m."""
    half = rotary_dim // 2
    rows = [(m, 0.0), (0.0, m), (-m, 0.0)]
    t = np.zeros((3, rotary_dim), dtype=np.float32)
    for p, (c, s) in enumerate(rows):
        t[p, :half] = c
        t[p, half:] = s
    return t


def _vals(a, dtype="bf16"):
    return bf16.to_f32(a, dtype).reshape(a.shape)


@pytest.mark.parametrize("m", [1.0, 2.0, 0.5])
@pytest.mark.parametrize("neox", [True, False])
def test_quarter_turns_are_exact(m, neox):
    rng = np.random.default_rng(0)
    dim = 8
    k, v = _pool(rng, dim=dim, layers=1)
    src_rows = k[0][[1, 2, 3]].copy()
    table = _exact_table(dim, m)
    # token 0: 0 -> 90deg, token 1: 90deg -> 0, token 2: 90deg -> 180deg
    rp.reposition_kv_layers(k, v, [1, 2, 3], [5, 6, 7], [[0, 1], [1, 0], [1, 2]], table,
                            dtype="bf16", is_neox_style=neox)
    half = dim // 2
    idx1 = np.arange(half) if neox else 2 * np.arange(half)
    idx2 = idx1 + half if neox else idx1 + 1
    x = _vals(src_rows)
    x1, x2 = x[..., idx1], x[..., idx2]
    y = _vals(k[0][[5, 6, 7]])
    # +90 degrees: (x1, x2) -> (-x2, x1); -90 degrees: (x1, x2) -> (x2, -x1)
    np.testing.assert_array_equal(y[0][..., idx1], -x2[0])
    np.testing.assert_array_equal(y[0][..., idx2], x1[0])
    np.testing.assert_array_equal(y[1][..., idx1], x2[1])
    np.testing.assert_array_equal(y[1][..., idx2], -x1[1])
    np.testing.assert_array_equal(y[2][..., idx1], -x2[2])
    np.testing.assert_array_equal(y[2][..., idx2], x1[2])


def test_same_position_keeps_bits_even_when_the_math_would_not():
    # fp32 storage: there the arithmetic round trip visibly perturbs the bits
    rng = np.random.default_rng(1)
    k, v = _pool(rng, dim=8, layers=2, dtype="f32")
    # a table whose round trip is inexact (|cos, sin| != 1)
    table = np.full((4, 8), 0.3, dtype=np.float32)
    table[2, :4], table[2, 4:] = 0.71, 0.33
    before = [x[[1, 2]].copy() for x in k]
    rp.reposition_kv_layers(k, v, [1, 2], [4, 5], [[2, 2], [3, 3]], table, dtype="f32")
    for layer, b in zip(k, before):
        np.testing.assert_array_equal(layer[[4, 5]].view(np.uint32), b.view(np.uint32))
    # and the same rows through the arithmetic path do change
    y1, _ = rp.rotate_pairs(before[0][0, :, :4], before[0][0, :, 4:],
                            table[2, :4], table[2, 4:], table[2, :4], table[2, 4:])
    assert not np.array_equal(y1.view(np.uint32), before[0][0, :, :4].copy().view(np.uint32))


def test_plain_round_trip_within_two_ulp():
    rng = np.random.default_rng(2)
    dim, positions = 64, 4096
    inv = 1.0 / (10000.0 ** (np.arange(0, dim, 2, dtype=np.float32) / dim))
    ang = np.outer(np.arange(positions, dtype=np.float32), inv).astype(np.float32)
    table = np.concatenate((np.cos(ang), np.sin(ang)), axis=1).astype(np.float32)
    k, v = _pool(rng, slots=64, heads=4, dim=dim, layers=1)
    orig = k[0][1:21].copy()
    p = rng.integers(0, positions, size=20)
    q = rng.integers(0, positions, size=20)
    rp.reposition_kv_layers(k, v, np.arange(1, 21), np.arange(21, 41), np.stack([p, q], 1), table, dtype="bf16")
    rp.reposition_kv_layers(k, v, np.arange(21, 41), np.arange(41, 61), np.stack([q, p], 1), table, dtype="bf16")
    back = _vals(k[0][41:61])
    ref = _vals(orig)
    # each bf16 store rounds relative to the pair's magnitude (the partner
    # component leaks into each output): two stores -> within 2 bf16 ulp of it
    h = dim // 2
    pair = np.maximum(np.abs(ref[..., :h]), np.abs(ref[..., h:]))
    pair = np.concatenate((pair, pair), axis=-1)
    assert np.all(np.abs(back - ref) <= 2 * pair * 2.0**-7)
    assert np.mean(back == ref) > 0.7


def test_matches_delta_rotation_in_float64_away_from_cancellation():
    rng = np.random.default_rng(3)
    dim = 16
    k, v = _pool(rng, slots=32, heads=2, dim=dim, layers=1)
    m = 1.3466
    inv = 1.0 / (150000.0 ** (np.arange(0, dim, 2) / dim))
    ang = np.outer(np.arange(64), inv)
    table = (np.concatenate((np.cos(ang), np.sin(ang)), 1) * m).astype(np.float32)
    old = rng.integers(0, 64, size=10)
    new = rng.integers(0, 64, size=10)
    x = _vals(k[0][1:11]).astype(np.float64)
    rp.reposition_kv_layers(k, v, np.arange(1, 11), np.arange(11, 21), np.stack([old, new], 1), table, dtype="bf16")
    y = _vals(k[0][11:21]).astype(np.float64)
    h = dim // 2
    t64 = table.astype(np.float64)
    c = (t64[new, :h] * t64[old, :h] + t64[new, h:] * t64[old, h:]) / (t64[old, :h] ** 2 + t64[old, h:] ** 2)
    s = (t64[new, h:] * t64[old, :h] - t64[new, :h] * t64[old, h:]) / (t64[old, :h] ** 2 + t64[old, h:] ** 2)
    c, s = c[:, None, :], s[:, None, :]
    want1 = x[..., :h] * c - x[..., h:] * s
    want2 = x[..., h:] * c + x[..., :h] * s
    scale = np.maximum(np.abs(x[..., :h]), np.abs(x[..., h:]))
    assert np.all(np.abs(y[..., :h] - want1) <= scale * 2.0**-6 + 1e-6)
    assert np.all(np.abs(y[..., h:] - want2) <= scale * 2.0**-6 + 1e-6)


def test_tail_and_v_are_bitwise_and_skip_unmapped():
    rng = np.random.default_rng(4)
    k, v = _pool(rng, slots=10, heads=2, dim=16, layers=2)
    table = _exact_table(8, 1.0)
    k_before = [x.copy() for x in k]
    v_before = [x.copy() for x in v]
    # token 1 has an unmapped destination (0): skipped entirely with skip_unmapped
    rp.reposition_kv_layers(k, v, [1, 2], [6, 0], [[0, 1], [0, 1]], table, dtype="bf16",
                            skip_unmapped=True, rotary_dim=8)
    for l in range(2):
        np.testing.assert_array_equal(k[l][6, :, 8:], k_before[l][1, :, 8:])
        np.testing.assert_array_equal(v[l][6], v_before[l][1])
        np.testing.assert_array_equal(k[l][0], k_before[l][0])
        np.testing.assert_array_equal(v[l][0], v_before[l][0])
        untouched = [s for s in range(10) if s != 6]
        np.testing.assert_array_equal(k[l][untouched], k_before[l][untouched])


def test_f32_and_f16_storage():
    rng = np.random.default_rng(5)
    for dtype in ("f32", "f16"):
        k, v = _pool(rng, dim=8, layers=1, dtype=dtype)
        table = _exact_table(8, 2.0)
        x = _vals(k[0][1], dtype)
        rp.reposition_kv_layers(k, v, [1], [2], [[0, 1]], table, dtype=dtype)
        y = _vals(k[0][2], dtype)
        np.testing.assert_array_equal(y[:, :4], -x[:, 4:])
        np.testing.assert_array_equal(y[:, 4:], x[:, :4])


# -- known answers for the fp32 operation order ---------------------------
#
# tests/golden/reposition_kat.npz holds 64 (x1, x2, old, new) cases on the
# GPT-OSS YaRN table whose bf16 result under the reference order
# (context_reposition.py:92-102, every operation rounded, no FMA) differs
# from a delta-angle rotation, from dividing each product before the sum and
# from fused multiply-adds.  The expected bits come from exact rational
# arithmetic (tests/exact_fp.py), not from numpy.

def test_kat_fixture_is_exact_and_discriminating():
    for c in range(len(KAT["old"])):
        args = [int(KAT[f][c]) for f in ("x1_bits", "x2_bits", "co_bits", "so_bits", "cn_bits", "sn_bits")]
        ref = ex.rotate_bf16_bits("two_step", *args)
        assert ref == tuple(int(b) for b in KAT["two_step_bits"][c])
        for form in KAT_VARIANTS:
            got = ex.rotate_bf16_bits(form, *args)
            assert got == tuple(int(b) for b in KAT[f"{form}_bits"][c])
            assert got != ref, (c, form)


def test_exact_rounding_against_the_format_definition():
    # spot checks of the rounding helper itself: ties to even, subnormals,
    # exactly representable values, and agreement with numpy's IEEE float32
    tie_up = Fraction(1) + Fraction(3, 2**24)  # halfway between 1+2^-23 and 1+2^-22
    assert ex.f32(tie_up) == 1 + Fraction(2, 2**23)
    tie_down = Fraction(1) + Fraction(1, 2**24)  # halfway between 1 and 1+2^-23
    assert ex.f32(tie_down) == 1
    assert ex.f32(Fraction(3, 2**150)) == Fraction(2, 2**149)  # 1.5 quanta -> 2 (even)
    assert ex.f32(Fraction(1, 2**150)) == 0  # half the smallest subnormal -> 0 (even)
    assert ex.round_binary(Fraction(1) + Fraction(1, 2**8), ex.BF16) == 1
    assert ex.round_binary(Fraction(1) + Fraction(3, 2**8), ex.BF16) == 1 + Fraction(2, 2**7)
    rng = np.random.default_rng(7)
    a = rng.standard_normal(200).astype(np.float32)
    b = rng.standard_normal(200).astype(np.float32) + 2
    for op in (np.multiply, np.add, np.subtract, np.divide):
        got = op(a, b)
        for i in range(len(a)):
            x, y = Fraction(float(a[i])), Fraction(float(b[i]))
            exact = {np.multiply: x * y, np.add: x + y, np.subtract: x - y, np.divide: x / y}[op]
            assert ex.f32(exact) == Fraction(float(got[i]))


@pytest.mark.parametrize("neox", [True, False])
def test_oracle_matches_exact_operation_order(neox):
    k, v, src, dst, pairs, table = kat_pool(neox)
    v_before = v[0].copy()
    rp.reposition_kv_layers(k, v, src, dst, pairs, table, dtype="bf16", is_neox_style=neox)
    np.testing.assert_array_equal(k[0][dst], kat_expected("two_step", neox))
    np.testing.assert_array_equal(v[0][dst], v_before[src])


def _planted(form):
    """numpy float32 statements of the three variants, planted in place of
    the oracle's rotation."""
    f = np.float32

    def fma(a, b, c):
        return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(f)

    def rotate(x1, x2, co, so, cn, sn):
        x1, x2, co, so, cn, sn = (np.asarray(a, dtype=f) for a in (x1, x2, co, so, cn, sn))
        s = co * co + so * so
        if form == "delta_angle":
            cd = (cn * co + sn * so) / s
            sd = (sn * co - cn * so) / s
            return x1 * cd - x2 * sd, x2 * cd + x1 * sd
        if form == "per_term_division":
            u1 = (x1 * co) / s + (x2 * so) / s
            u2 = (x2 * co) / s - (x1 * so) / s
            return u1 * cn - u2 * sn, u2 * cn + u1 * sn
        s = fma(co, co, so * so)
        u1 = fma(x1, co, x2 * so) / s
        u2 = fma(x2, co, -(x1 * so)) / s
        return fma(u1, cn, -(u2 * sn)), fma(u2, cn, u1 * sn)

    return rotate


@pytest.mark.parametrize("form", KAT_VARIANTS)
def test_known_answers_reject_planted_variants(form, monkeypatch):
    monkeypatch.setattr(rp, "rotate_pairs", _planted(form))
    k, v, src, dst, pairs, table = kat_pool(True)
    rp.reposition_kv_layers(k, v, src, dst, pairs, table, dtype="bf16")
    got = k[0][dst]
    assert not np.array_equal(got, kat_expected("two_step"))
    # the planted form reproduces its own exact known answers on most cases
    # (the float64 emulation of an FMA can double-round)
    assert np.mean(np.all(got == kat_expected(form), axis=(1, 2))) > 0.9
