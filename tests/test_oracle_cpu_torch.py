"""Pins oracle.cpu_torch (the vectorised torch-CPU baseline) to the exact
known answers and to oracle.reposition, bit for bit."""

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import cpu_torch
from oracle import reposition as rp
from reposition_kat import kat_expected, kat_pool

TORCH = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _to_torch(a, dtype):
    if dtype == "f32":
        return torch.from_numpy(np.ascontiguousarray(a).view(np.float32).copy())
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16).copy()).view(TORCH[dtype])


def _to_storage(t, dtype):
    if dtype == "f32":
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


@pytest.mark.parametrize("neox", [True, False])
def test_exact_known_answers(neox):
    k, v, src, dst, pairs, table = kat_pool(neox)
    kt, vt = [_to_torch(k[0], "bf16")], [_to_torch(v[0], "bf16")]
    cpu_torch.reposition_kv_layers(kt, vt, src, dst, pairs, torch.from_numpy(table), is_neox_style=neox)
    np.testing.assert_array_equal(_to_storage(kt[0], "bf16")[dst], kat_expected("two_step", neox))
    np.testing.assert_array_equal(_to_storage(vt[0], "bf16")[dst], v[0][src])


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("neox,rotary", [(True, 64), (False, 64), (True, 32), (False, 16)])
def test_matches_numpy_oracle(dtype, neox, rotary):
    rng = np.random.default_rng(rotary + len(dtype))
    layers, slots, heads, dim, moved = 3, 300, 4, 64, 120
    k = [bf16.from_f32(rng.standard_normal((slots, heads, dim)).astype(np.float32), dtype).reshape(slots, heads, dim)
         for _ in range(layers)]
    v = [bf16.from_f32(rng.standard_normal((slots, heads, dim)).astype(np.float32), dtype).reshape(slots, heads, dim)
         for _ in range(layers)]
    perm = rng.permutation(np.arange(1, slots))
    src, dst = perm[:moved], perm[moved : 2 * moved]
    dst[::13] = 0  # unmapped destinations, skipped with skip_unmapped
    old = rng.integers(0, 500, moved)
    new = rng.integers(0, 500, moved)
    new[::5] = old[::5]
    pairs = np.stack((old, new), 1)
    ang = np.outer(np.arange(500), 1.0 / 150000.0 ** (np.arange(0, rotary, 2) / rotary))
    table = (np.concatenate((np.cos(ang), np.sin(ang)), 1) * 1.3466).astype(np.float32)
    kt = [_to_torch(x, dtype) for x in k]
    vt = [_to_torch(x, dtype) for x in v]
    rp.reposition_kv_layers(k, v, src, dst, pairs, table, dtype=dtype, is_neox_style=neox, rotary_dim=rotary,
                            skip_unmapped=True)
    cpu_torch.reposition_kv_layers(kt, vt, src, dst, pairs, torch.from_numpy(table), is_neox_style=neox,
                                   rotary_dim=rotary, skip_unmapped=True)
    for layer in range(layers):
        np.testing.assert_array_equal(_to_storage(kt[layer], dtype), k[layer])
        np.testing.assert_array_equal(_to_storage(vt[layer], dtype), v[layer])
