"""GPU: device parts of the P -> D handoff mirror -- active-slot gathers,
D-side destination allocation (fresh and borrowed owners, ownership state,
table row) and the Reposition of reused versions at new positions."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from akv_amd import binding, handoff
from akv_amd.rope import make_table
from oracle import reposition as rp

from helpers import storage_equal, to_storage
from test_handoff_host import _program

pytestmark = pytest.mark.gpu


def _pool(device, rows, width, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    table = torch.randint(1, 1 << 20, (rows, width), generator=g, device=device, dtype=torch.int32)

    def write(where, values):
        idx, cols = where
        table[idx, cols] = values.to(torch.int32)

    return SimpleNamespace(req_to_token=table, write=write)


def test_active_slot_gathers(device):
    for seed in range(10):
        prog, rng = _program(500 + seed)
        p = handoff.ContextTransferPlan.build(prog, device)
        n = len(prog.layout.positions)
        pool = _pool(device, 4, n + 16, seed)
        req = SimpleNamespace(kv=SimpleNamespace(req_pool_idx=2), context_decode_layout=p.decode,
                              context_program=prog)
        row = pool.req_to_token[2]
        raw = torch.from_numpy(p.decode.raw_indices.astype(np.int64)).to(device)
        assert torch.equal(p.slots(req, pool), row[raw])
        for window in (3, 17):
            start = p.swa_start(window)
            assert torch.equal(p.slots(req, pool, window=window), row[raw[start:]])
        for generated in (0, 5):
            end = n + generated
            want = torch.cat((row[raw], row[n:end]))
            assert torch.equal(handoff.request_active_slots(req, pool, end), want)
            window = 9
            lower = p.decode.next_position + generated - window
            start = int(np.searchsorted(p.decode.positions, lower))
            gen_start = n + max(0, lower - p.decode.next_position)
            want = torch.cat((row[raw[start:]], row[gen_start:end]))
            assert torch.equal(handoff.request_active_slots(req, pool, end, window=window), want)


def _req(prog, device, **kw):
    base = dict(kv=SimpleNamespace(req_pool_idx=1, kv_allocated_len=0), context_program=prog,
                context_recompute_program=None, context_decode_layout=None, context_exact_prefix_len=0)
    base.update(kw)
    return SimpleNamespace(**base)


def test_destination_allocation_fresh_and_borrowed(device):
    for seed in range(10):
        prog, rng = _program(600 + seed)
        n = len(prog.layout.positions)
        keep = prog.layout.keep_mask.numpy()
        count = int(keep.sum())
        pool = _pool(device, 3, n + 8, seed)
        alloc = SimpleNamespace(device=device, alloc=lambda k: torch.arange(50_000, 50_000 + k, device=device))
        # every active version fresh
        req = _req(prog, device)
        slots = handoff.allocate_context_destination(req, alloc, pool)
        torch.cuda.synchronize()
        assert torch.equal(slots.cpu(), torch.arange(50_000, 50_000 + count))
        row = np.full(n, -1, dtype=np.int64)
        row[np.flatnonzero(keep)] = np.arange(50_000, 50_000 + count)
        assert np.array_equal(req.context_state.terminal_slots().cpu().numpy(), row)
        assert np.array_equal(pool.req_to_token[1, :n].cpu().numpy(), row)
        assert req.kv.kv_allocated_len == n and bool(req.context_state.owned.all())
        # D's own match borrowed where it is at the right position
        matched = int(rng.integers(1, n))
        prefix = torch.from_numpy(rng.permutation(np.arange(900_000, 900_000 + matched))).to(device)
        req = _req(prog, device, prefix_indices=prefix, context_resident=None,
                   context_source_positions=torch.from_numpy(prog.layout.positions.numpy()[:matched].copy()),
                   context_exact_prefix_len=matched)
        p = handoff.transfer_plan(req, device)
        req.context_decode_reuse = handoff.ContextDecodeReuse.build(req, p)
        reuse = req.context_decode_reuse
        slots = handoff.allocate_context_destination(req, alloc, pool).cpu().numpy()
        raw = p.decode.raw_indices
        fresh = iter(range(50_000, 50_000 + reuse.allocation_count))
        for i in range(count):
            want = int(prefix[raw[i]]) if reuse.borrowed[i] else next(fresh)
            assert slots[i] == want, (seed, i)
        assert np.array_equal(req.context_state.owned.numpy(), ~reuse.borrowed)
        private = raw[~reuse.borrowed]
        assert req.context_exact_prefix_len == (min(matched, int(private[0])) if len(private) else matched)


def test_reused_versions_are_repositioned(device):
    prog, rng = _program(700)
    n = len(prog.layout.positions)
    heads, dim, slots_total, positions = 2, 64, 4000, 512
    gen = torch.Generator().manual_seed(7)
    table = make_table("yarn", dim, positions, base=150000.0, factor=32.0, original_max=4096).to(device)
    kv = [(torch.randn((slots_total, heads, dim), generator=gen).to(torch.bfloat16).to(device),
           torch.randn((slots_total, heads, dim), generator=gen).to(torch.bfloat16).to(device)) for _ in range(2)]
    modules = [SimpleNamespace(attn=SimpleNamespace(layer_id=i, sliding_window_size=-1),
                               rotary_emb=SimpleNamespace(cos_sin_cache=table, rotary_dim=dim, is_neox_style=True))
               for i in range(2)]
    tr = SimpleNamespace(translate_full_attn_ids=lambda x: x, sliding_window_write_loc_for=lambda x: None)
    b = binding.ContextModelBinding(SimpleNamespace(modules=lambda: iter(modules)),
                                    SimpleNamespace(get_kv_buffer=lambda i: kv[i]), tr, page_size=1)
    matched = n
    prefix = torch.from_numpy(rng.permutation(np.arange(1, 2000))[:matched].astype(np.int64)).to(device)
    req = _req(prog, device, prefix_indices=prefix, context_resident=None,
               context_source_positions=torch.from_numpy(prog.layout.birth_positions.numpy()[:matched].copy()),
               context_exact_prefix_len=matched // 2)
    p = handoff.transfer_plan(req, device)
    req.context_decode_reuse = reuse = handoff.ContextDecodeReuse.build(req, p)
    assert len(reuse.copy_indices) > 0
    pool = _pool(device, 2, n + 8, 0)
    alloc = SimpleNamespace(device=device, alloc=lambda k: torch.arange(2000, 2000 + k, device=device))
    handoff.allocate_context_destination(req, alloc, pool)
    src = prefix.cpu().numpy()[p.decode.raw_indices[reuse.copy_indices]].astype(np.int32)
    dst = req.context_state.slots.cpu().numpy()[reuse.copy_indices].astype(np.int32)
    want = []
    for k, v in kv:
        kn, vn = [to_storage(k)], [to_storage(v)]
        rp.reposition_kv_layers(kn, vn, src, dst, reuse.position_pairs.numpy(), to_storage(table), dtype="bf16",
                                cos_sin_dtype="f32", is_neox_style=True, rotary_dim=dim)
        want.append((kn[0], vn[0]))
    print(f"reposition of {len(src)} reused versions", flush=True)
    handoff.materialize_decode_reuse(req, SimpleNamespace(context_model_binding=b))
    torch.cuda.synchronize()
    for (k, v), (wk, wv) in zip(kv, want):
        assert storage_equal(to_storage(k), wk) and storage_equal(to_storage(v), wv)
