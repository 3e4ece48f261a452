"""GPU: the layer binding of the Context prefill (``akv_amd.binding``).

A hybrid model -- full-attention layers in two shapes and sliding-window
layers in a separate SWA pool reached through an index translator -- is
bound once; ``reposition_existing`` (one launch per compatible group) and
the per-layer copies of ``ContextPrefillInput.bind`` must move exactly what
the oracle moves at the translated slots, leave unmapped SWA slots alone,
and hand each layer the attention metadata of its own pool."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from akv_amd import binding
from akv_amd.context_attention import ContextAttentionPlan, ContextSequence
from akv_amd.rope import make_table
from oracle import reposition as rp

from helpers import storage_equal, to_storage

pytestmark = pytest.mark.gpu

FULL_SLOTS, SWA_SLOTS, POSITIONS = 600, 400, 256


class Translator:
    """virtual full id -> physical full id (a permutation); physical full id
    -> SWA slot (0 where the SWA pool holds no copy)."""

    def __init__(self, device, rng, separate_swa=True):
        self.v2p = torch.from_numpy(np.r_[0, 1 + rng.permutation(FULL_SLOTS - 1)].astype(np.int64)).to(device)
        swa = np.zeros(FULL_SLOTS, dtype=np.int64)
        mapped = rng.choice(np.arange(1, FULL_SLOTS), size=SWA_SLOTS - 1, replace=False)
        swa[mapped] = np.arange(1, SWA_SLOTS)
        self.full_to_swa = torch.from_numpy(swa).to(device) if separate_swa else None

    def translate_full_attn_ids(self, ids):
        return self.v2p[ids.long()]

    def sliding_window_write_loc_for(self, ids):
        return None if self.full_to_swa is None else self.full_to_swa[ids.long()]


def _model(device, separate_swa=True):
    g = torch.Generator().manual_seed(0)
    table64 = make_table("yarn", 64, POSITIONS, base=150000.0, factor=32.0, original_max=4096).to(device)
    table32 = make_table("plain", 32, POSITIONS, base=10000.0).to(device)
    specs = [  # (layer_id, window, heads, dim, rotary table)
        (0, -1, 2, 64, table64), (1, 128, 2, 64, table64), (2, -1, 2, 64, table64), (3, 128, 2, 64, table64),
        (4, -1, 4, 64, table32), (5, -1, 4, 64, table32),
    ]
    buffers, modules = {}, []
    for lid, window, h, d, table in specs:
        slots = SWA_SLOTS if (window > -1 and separate_swa) else FULL_SLOTS
        k = torch.randn((slots, h, d), generator=g).to(torch.bfloat16).to(device)
        v = torch.randn((slots, h, d), generator=g).to(torch.bfloat16).to(device)
        buffers[lid] = (k, v)
        modules.append(SimpleNamespace(
            attn=SimpleNamespace(layer_id=lid, sliding_window_size=window),
            rotary_emb=SimpleNamespace(cos_sin_cache=table, rotary_dim=table.shape[1], is_neox_style=True)))
    modules.append(SimpleNamespace(attn=None))  # a non-attention module is skipped
    model = SimpleNamespace(modules=lambda: iter(modules))
    pool = SimpleNamespace(get_kv_buffer=lambda lid: buffers[lid])
    return model, pool, buffers, specs


def _expected(buffers, specs, src_full, dst_full, pairs, to_swa):
    """Oracle result per layer at the physical slots each pool uses."""
    want = {}
    for lid, window, h, d, table in specs:
        k, v = buffers[lid]
        k_np, v_np = [to_storage(k)], [to_storage(v)]
        src, dst, skip = src_full, dst_full, False
        if window > -1 and to_swa is not None:
            src, dst, skip = to_swa[src_full], to_swa[dst_full], True
        rp.reposition_kv_layers(k_np, v_np, src.astype(np.int32), dst.astype(np.int32), pairs,
                                to_storage(table), dtype="bf16", cos_sin_dtype="f32", is_neox_style=True,
                                skip_unmapped=skip, rotary_dim=table.shape[1])
        want[lid] = (k_np[0], v_np[0])
    return want


def _copies(rng, n):
    perm = rng.permutation(np.arange(1, FULL_SLOTS))
    pairs = np.stack((rng.integers(0, POSITIONS, n), rng.integers(0, POSITIONS, n)), 1).astype(np.int32)
    return perm[:n].astype(np.int32), perm[n : 2 * n].astype(np.int32), pairs


@pytest.mark.parametrize("separate_swa", [True, False])
def test_reposition_existing_groups_and_translates(device, separate_swa):
    rng = np.random.default_rng(1)
    model, pool, buffers, specs = _model(device, separate_swa)
    tr = Translator(device, rng, separate_swa)
    b = binding.ContextModelBinding(model, pool, tr, page_size=1)
    assert b.launches == 3 and b.has_swa  # full 2x64, SWA 2x64, full 4x64 (own table)
    src, dst, pairs = _copies(rng, 150)
    v2p = tr.v2p.cpu().numpy()
    to_swa = None if tr.full_to_swa is None else tr.full_to_swa.cpu().numpy()
    want = _expected(buffers, specs, v2p[src], v2p[dst], pairs, to_swa)
    print(f"reposition_existing separate_swa={separate_swa}", flush=True)
    b.reposition_existing(torch.from_numpy(src).to(device), torch.from_numpy(dst).to(device),
                          torch.from_numpy(pairs).to(device))
    torch.cuda.synchronize()
    for lid, (k, v) in buffers.items():
        assert storage_equal(to_storage(k), want[lid][0]), f"K layer {lid}"
        assert storage_equal(to_storage(v), want[lid][1]), f"V layer {lid}"


def test_prefill_input_bind_per_layer_copies_and_metadata(device):
    rng = np.random.default_rng(2)
    model, pool, buffers, specs = _model(device)
    tr = Translator(device, rng)
    b = binding.ContextModelBinding(model, pool, tr, page_size=1)
    seqs = [ContextSequence.ordinary(40, 9), ContextSequence.ordinary(0, 30)]
    plan = ContextAttentionPlan.merge(seqs)
    occ = torch.from_numpy(rng.permutation(np.arange(1, FULL_SLOTS))[: plan.occurrence_count]).to(device)
    src, dst, pairs = _copies(rng, 90)
    inp = binding.ContextPrefillInput(plan, occ, torch.from_numpy(src).to(device), torch.from_numpy(dst).to(device),
                                      torch.from_numpy(pairs).to(device), b)
    meta = inp.bind()
    v2p = tr.v2p.cpu().numpy()
    to_swa = tr.full_to_swa.cpu().numpy()
    want = _expected(buffers, specs, v2p[src], v2p[dst], pairs, to_swa)
    print("per-layer copies of a bound prefill input", flush=True)
    for lid in sorted(meta.layer_copies):
        meta.layer_copies[lid].apply()
    torch.cuda.synchronize()
    for lid, (k, v) in buffers.items():
        assert storage_equal(to_storage(k), want[lid][0]), f"K layer {lid}"
        assert storage_equal(to_storage(v), want[lid][1]), f"V layer {lid}"
    # metadata: full layers read translated slots, SWA layers their SWA slots
    _, _, occurrences, _, _ = meta.full.cpu_fields
    full_phys = v2p[occ.cpu().numpy()]
    assert np.array_equal(meta.full.kv_indices.cpu().numpy(), full_phys[occurrences])
    assert np.array_equal(meta.sliding_window.kv_indices.cpu().numpy(), to_swa[full_phys][occurrences])
    swa_layer = SimpleNamespace(sliding_window_size=128)
    assert meta.for_layer(swa_layer) is meta.sliding_window
    assert meta.for_layer(SimpleNamespace(sliding_window_size=None)) is meta.full
    # concatenation keeps every field of both inputs in order
    both = binding.ContextPrefillInput.concatenate([inp, inp])
    assert both.attention_plan.occurrence_count == 2 * plan.occurrence_count
    assert torch.equal(both.copy_sources, torch.cat([inp.copy_sources] * 2))


def test_binding_validation(device):
    model, pool, buffers, specs = _model(device)
    tr = Translator(device, np.random.default_rng(3))
    with pytest.raises(ValueError, match="requires page_size=1"):
        binding.ContextModelBinding(model, pool, tr, page_size=16)
    bad = SimpleNamespace(modules=lambda: iter([SimpleNamespace(
        attn=SimpleNamespace(layer_id=0, sliding_window_size=-1),
        rotary_emb=SimpleNamespace(cos_sin_cache=torch.zeros((8, 63), device=device), rotary_dim=63,
                                   is_neox_style=True))]))
    with pytest.raises(ValueError, match="native NHD KV and valid native rotary_dim"):
        binding.ContextModelBinding(bad, pool, tr, page_size=1)
    with pytest.raises(ValueError, match="unique native attention layers"):
        binding.ContextModelBinding(SimpleNamespace(modules=lambda: iter([])), pool, tr, page_size=1)
    plan = ContextAttentionPlan.merge([ContextSequence.ordinary(2, 2)])
    z = torch.zeros(3, dtype=torch.int64, device=device)
    inp = binding.ContextPrefillInput(plan, torch.arange(4, device=device), z, z, z.view(-1, 1), None)
    with pytest.raises(ValueError, match="aligned int32 metadata"):
        inp.bind()
