"""Pins oracle.reposition with closed forms a plausible mistake cannot pass.

Exact tables (cos/sin in {-m, 0, m}, m a power of two) make every rotation
exact, so a swapped sign, a cos/sin half swap, a wrong pair index, a dropped
division by cos^2 + sin^2 or a transposed operand gives a different answer.
"""

import numpy as np
import pytest

from oracle import bf16
from oracle import reposition as rp


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
