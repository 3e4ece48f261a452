"""GPU: one Reposition launch per compatible group of a hybrid model's layers.

Full-attention layers in two shapes (one with a partial rotary width) and
sliding-window layers whose pool is reached through a full -> SWA slot map
(0 where the SWA pool holds no copy): every group is one
``reposition_kv_layers`` launch over its layers' pointer tables, and every
layer must end bit-equal to the oracle at the slots its pool uses, with
unmapped SWA slots left alone.  This is the call pattern of the
reference's model binding (``context_backend.py:373-472``), played by the
test harness."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from akv_amd.rope import make_table
from oracle import reposition as rp

from harness import reposition_groups
from helpers import storage_equal, to_storage

pytestmark = pytest.mark.gpu

FULL_SLOTS, SWA_SLOTS, POSITIONS = 600, 400, 256


def _model(device, rng, separate_swa):
    g = torch.Generator().manual_seed(0)
    yarn = make_table("yarn", 64, POSITIONS, base=150000.0, factor=32.0, original_max=4096).to(device)
    plain = make_table("plain", 32, POSITIONS, base=10000.0).to(device)
    to_swa = None
    if separate_swa:
        m = np.zeros(FULL_SLOTS, dtype=np.int64)
        m[rng.choice(np.arange(1, FULL_SLOTS), size=SWA_SLOTS - 1, replace=False)] = np.arange(1, SWA_SLOTS)
        to_swa = torch.from_numpy(m).to(device)
    specs = [  # (sliding window, heads, head dim, rotary table)
        (False, 2, 64, yarn), (True, 2, 64, yarn), (False, 2, 64, yarn), (True, 2, 64, yarn),
        (False, 4, 64, plain), (False, 4, 64, plain),
    ]
    layers = []
    for swa, h, d, table in specs:
        slots = SWA_SLOTS if (swa and separate_swa) else FULL_SLOTS
        k = torch.randn((slots, h, d), generator=g).to(torch.bfloat16).to(device)
        v = torch.randn((slots, h, d), generator=g).to(torch.bfloat16).to(device)
        layers.append(SimpleNamespace(k=k, v=v, table=table, is_neox=True, rotary_dim=table.shape[1],
                                      to_slots=to_swa if swa else None))
    return layers


def _expected(layers, src, dst, pairs):
    want = []
    for layer in layers:
        k_np, v_np = [to_storage(layer.k)], [to_storage(layer.v)]
        s, d, skip = src, dst, False
        if layer.to_slots is not None:
            m = layer.to_slots.cpu().numpy()
            s, d, skip = m[src], m[dst], True
        rp.reposition_kv_layers(k_np, v_np, s.astype(np.int32), d.astype(np.int32), pairs, to_storage(layer.table),
                                dtype="bf16", cos_sin_dtype="f32", is_neox_style=True, skip_unmapped=skip,
                                rotary_dim=layer.rotary_dim)
        want.append((k_np[0], v_np[0]))
    return want


@pytest.mark.parametrize("separate_swa", [True, False])
def test_groups_translate_and_match_oracle(device, separate_swa):
    rng = np.random.default_rng(1)
    layers = _model(device, rng, separate_swa)
    perm = rng.permutation(np.arange(1, FULL_SLOTS))
    n = 150
    src, dst = perm[:n].astype(np.int32), perm[n : 2 * n].astype(np.int32)
    pairs = np.stack((rng.integers(0, POSITIONS, n), rng.integers(0, POSITIONS, n)), 1).astype(np.int32)
    want = _expected(layers, src, dst, pairs)
    print(f"layer groups separate_swa={separate_swa}", flush=True)
    launches = reposition_groups(layers, torch.from_numpy(src).to(device), torch.from_numpy(dst).to(device),
                                 torch.from_numpy(pairs).to(device))
    torch.cuda.synchronize()
    # full 2x64, full 4x64 with its own table, and (separate pool) the SWA layers
    assert launches == (3 if separate_swa else 2)
    for i, layer in enumerate(layers):
        assert storage_equal(to_storage(layer.k), want[i][0]), f"K layer {i}"
        assert storage_equal(to_storage(layer.v), want[i][1]), f"V layer {i}"


@pytest.mark.parametrize("seed", range(8))
def test_random_hybrid_models(device, seed):
    # seeded random hybrid models: 2-12 layers, sliding-window layers in a
    # separate or the shared pool, 1-4 heads of 32-128 dims, YaRN or plain
    # tables with full or partial rotary widths
    rng = np.random.default_rng(1400 + seed)
    g = torch.Generator().manual_seed(1400 + seed)
    tables = {("yarn", 128): make_table("yarn", 128, POSITIONS, base=150000.0, factor=32.0, original_max=4096),
              ("yarn", 64): make_table("yarn", 64, POSITIONS, base=150000.0, factor=32.0, original_max=4096),
              ("plain", 32): make_table("plain", 32, POSITIONS, base=10000.0),
              ("plain", 16): make_table("plain", 16, POSITIONS, base=10000.0)}
    tables = {k: t.to(device) for k, t in tables.items()}
    separate_swa = bool(rng.integers(0, 2))
    to_swa = None
    if separate_swa:
        m = np.zeros(FULL_SLOTS, dtype=np.int64)
        m[rng.choice(np.arange(1, FULL_SLOTS), size=SWA_SLOTS - 1, replace=False)] = np.arange(1, SWA_SLOTS)
        to_swa = torch.from_numpy(m).to(device)
    layers, keys = [], set()
    for _ in range(int(rng.integers(2, 13))):
        swa = bool(rng.integers(0, 2))
        h, d = int(rng.choice([1, 2, 4])), int(rng.choice([32, 64, 128]))
        fits = [k for k in tables if k[1] <= d]
        tkey = fits[int(rng.integers(0, len(fits)))]
        slots = SWA_SLOTS if (swa and separate_swa) else FULL_SLOTS
        k = torch.randn((slots, h, d), generator=g).to(torch.bfloat16).to(device)
        v = torch.randn((slots, h, d), generator=g).to(torch.bfloat16).to(device)
        layers.append(SimpleNamespace(k=k, v=v, table=tables[tkey], is_neox=True, rotary_dim=tkey[1],
                                      to_slots=to_swa if (swa and separate_swa) else None))
        keys.add((h, d, tkey, swa and separate_swa))
    perm = rng.permutation(np.arange(1, FULL_SLOTS))
    n = int(rng.integers(1, FULL_SLOTS // 2))
    src, dst = perm[:n].astype(np.int32), perm[n : 2 * n].astype(np.int32)
    pairs = np.stack((rng.integers(0, POSITIONS, n), rng.integers(0, POSITIONS, n)), 1).astype(np.int32)
    want = _expected(layers, src, dst, pairs)
    print(f"hybrid random {seed}: {len(layers)} layers, separate_swa={separate_swa}, n={n}", flush=True)
    launches = reposition_groups(layers, torch.from_numpy(src).to(device), torch.from_numpy(dst).to(device),
                                 torch.from_numpy(pairs).to(device))
    torch.cuda.synchronize()
    assert launches == len(keys)
    for i, layer in enumerate(layers):
        assert storage_equal(to_storage(layer.k), want[i][0]), f"K layer {i}"
        assert storage_equal(to_storage(layer.v), want[i][1]), f"V layer {i}"
