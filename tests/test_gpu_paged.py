"""GPU parity of page-granular compaction with copy-on-write (page size 16).

Tables, copy lists, released pages and page tables bit-exact against the
paging oracle; K re-rotated bit-exact and V moved bit for bit into fresh
pages; shared prefix pages and every other slot left untouched.  With page
size 1 the paged kernel reproduces ``akv_compact_rows``.
"""

import dataclasses

import numpy as np
import pytest
import torch

from akv_amd import ops, synth, tables
from oracle import paging as pg
from oracle import reposition as rp

from helpers import storage_equal, to_storage

pytestmark = pytest.mark.gpu


def _table_for(rows, width, device, order):
    table = torch.full((len(rows) + 3, width), -7, dtype=torch.int32)
    for b, r in enumerate(rows):
        table[order[b], : len(r)] = torch.from_numpy(r)
    return table.to(device)


def _run_groups(w, a, layouts, table, req_rows, device, pool=None, cos_sin=None, row_pointers=None):
    """Compact (and reposition) group by group; return per-request device outputs."""
    P = w.page_size
    got = {}
    for g in a.groups:
        g = list(g)
        inp = tables.pack_paged_inputs([layouts[b] for b in g], P, device)
        out = tables.allocate_paged_outputs(inp, device)
        fresh = np.concatenate([a.fresh_pages[b] for b in g]).astype(np.int32)
        rows = torch.tensor([req_rows[b] for b in g], dtype=torch.int64, device=device)
        tables.compact_pages(inp, table, rows, torch.from_numpy(fresh).to(device), out,
                             row_pointers=row_pointers)
        if pool is not None:
            ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src,
                                     out.copy_dst, out.copy_pairs, cos_sin)
        host = {k: getattr(out, k).cpu().numpy() for k in
                ("copy_src", "copy_dst", "copy_pairs", "released_pages", "page_table", "raw_indices",
                 "active_positions")}
        bases = inp.bases.cpu().numpy()
        for j, b in enumerate(g):
            got[b] = {
                "copy_source_slots": host["copy_src"][bases[2, j] : bases[2, j + 1]],
                "copy_destination_slots": host["copy_dst"][bases[2, j] : bases[2, j + 1]],
                "copy_position_pairs": host["copy_pairs"][bases[2, j] : bases[2, j + 1]],
                "released_pages": host["released_pages"][bases[5, j] : bases[5, j + 1]],
                "page_table": host["page_table"][bases[4, j] : bases[4, j + 1]],
                "raw_indices": host["raw_indices"][bases[1, j] : bases[1, j + 1]],
                "active_positions": host["active_positions"][bases[1, j] : bases[1, j + 1]],
            }
    return got


def _check_tables(w, a, layouts, got, table, order):
    table_np = table.cpu().numpy()
    for b, lay in enumerate(layouts):
        want = pg.compact_pages(a.birth_rows[b], lay.keep_mask, lay.birth_positions, lay.positions,
                                a.fresh_pages[b], w.page_size)
        n = w.lengths[b]
        np.testing.assert_array_equal(table_np[order[b], :n], want["terminal_row"], err_msg=f"row {b}")
        assert (table_np[order[b], n:] == -7).all()
        for key, value in got[b].items():
            np.testing.assert_array_equal(value, np.asarray(want[key]).astype(value.dtype),
                                          err_msg=f"{key} of request {b}")


@pytest.mark.parametrize("name,groups", [("llama3-cow-small", None), ("llama3-cow-small", "quarters"),
                                         ("llama3-cow-16", "quarters")])
def test_shared_prefix_cow_bit_exact(device, name, groups):
    # the full-size workload keeps every token count and page of the 16
    # requests but 2 of the 32 layers (a 13 GiB pool instead of 214 GiB)
    w = dataclasses.replace(synth.workload(name), model=synth.LLAMA3_8B_2L)
    B = w.n_requests
    split = None if groups is None else [range(i, i + 4) for i in range(0, B, 4)]
    a = synth.assign_pages(w, split)
    layouts = synth.compile_layouts(w)
    P = w.page_size
    pool = synth.make_pool(w.model, a.pool_pages * P, device, seed=4, generate_on_device=True)
    cos_sin = synth.rope_table(w, device)
    k_before = [t.clone() for t in pool.k]
    v_before = [t.clone() for t in pool.v]
    order = np.random.default_rng(0).permutation(B + 3)[:B]
    table = _table_for(a.birth_rows, max(w.lengths) + 5, device, order)
    print(f"cow: {B} requests, {a.pool_pages} pages, groups={len(a.groups)}", flush=True)
    got = _run_groups(w, a, layouts, table, order, device, pool, cos_sin)
    torch.cuda.synchronize()
    _check_tables(w, a, layouts, got, table, order)

    src = np.concatenate([got[b]["copy_source_slots"] for b in range(B)]).astype(np.int64)
    dst = np.concatenate([got[b]["copy_destination_slots"] for b in range(B)]).astype(np.int64)
    pairs = np.concatenate([got[b]["copy_position_pairs"] for b in range(B)])
    assert len(np.unique(dst)) == len(dst)
    src_d = torch.from_numpy(src).to(device)
    dst_d = torch.from_numpy(dst).to(device)
    untouched = torch.ones(a.pool_pages * P, dtype=torch.bool, device=device)
    untouched[dst_d] = False
    table_np = to_storage(cos_sin)
    # the oracle's K check runs on a seeded sample of the copies (all of them
    # would take minutes of CPU); unmoved-position copies are all in it
    rng = np.random.default_rng(1)
    same = np.flatnonzero(pairs[:, 0] == pairs[:, 1])
    sample = np.union1d(rng.choice(len(src), size=min(len(src), 6000), replace=False), same)
    s_src, s_dst = src_d[torch.from_numpy(sample).to(device)], dst_d[torch.from_numpy(sample).to(device)]
    for l in range(w.model.n_layers):
        # V bit for bit, every other slot (shared prefix pages included) unchanged
        assert torch.equal(pool.v[l][dst_d].view(torch.int16), v_before[l][src_d].view(torch.int16))
        assert torch.equal(pool.k[l][untouched].view(torch.int16), k_before[l][untouched].view(torch.int16))
        assert torch.equal(pool.v[l][untouched].view(torch.int16), v_before[l][untouched].view(torch.int16))
        # K against the oracle's two-step rotation
        m = len(sample)
        kk = [np.concatenate((to_storage(k_before[l][s_src]), np.zeros((m,) + pool.k[l].shape[1:], np.uint16)))]
        vv = [np.zeros_like(kk[0])]
        rp.reposition_kv_layers(kk, vv, np.arange(m), np.arange(m, 2 * m), pairs[sample], table_np, dtype="bf16")
        assert storage_equal(to_storage(pool.k[l][s_dst]), kk[0][m:]), f"layer {l}"


def test_cow_one_group_all_32_layers(device):
    """The full Llama-3-8B copy-on-write workload's first request group (4
    requests over the shared 8192-token prefix, 394,728 tokens) at all 32
    layers (a 92 GiB pool): tables bit-exact, V moved bit for bit and every
    other slot unchanged (per-layer checksums) in full, K against the
    torch-CPU restatement on a seeded sample of 6000 copies per layer (every
    same-position copy included)."""
    from oracle import cpu_torch

    full = synth.workload("llama3-cow-16")
    w = dataclasses.replace(full, lengths=full.lengths[:4], spans=full.spans[:4])
    assert w.model.n_layers == 32
    B = w.n_requests
    a = synth.assign_pages(w)
    layouts = synth.compile_layouts(w)
    P = w.page_size
    slots = a.pool_pages * P
    print(f"cow one group: {B} requests, {sum(w.lengths)} tokens, {a.pool_pages} pages, 32 layers", flush=True)
    pool = synth.make_pool(w.model, slots, device, seed=4, generate_on_device=True)
    cos_sin = synth.rope_table(w, device)
    order = np.arange(B)
    table = _table_for(a.birth_rows, max(w.lengths) + 5, device, order)
    # the copies' destinations are fresh pages: every other slot keeps its bits
    fresh = np.concatenate(a.fresh_pages).astype(np.int64)
    touched = torch.zeros(slots, dtype=torch.bool, device=device)
    if len(fresh):
        fresh_d = torch.from_numpy(fresh).to(device)
        touched.view(-1, P)[fresh_d] = True
    keep_sum = [t[~touched].view(torch.int16).to(torch.int64).sum().item() for t in pool.k + pool.v]
    got = _run_groups(w, a, layouts, table, order, device, pool, cos_sin)
    torch.cuda.synchronize()
    _check_tables(w, a, layouts, got, table, order)
    after_sum = [t[~touched].view(torch.int16).to(torch.int64).sum().item() for t in pool.k + pool.v]
    assert after_sum == keep_sum
    src = np.concatenate([got[b]["copy_source_slots"] for b in range(B)]).astype(np.int64)
    dst = np.concatenate([got[b]["copy_destination_slots"] for b in range(B)]).astype(np.int64)
    pairs = np.concatenate([got[b]["copy_position_pairs"] for b in range(B)])
    assert len(np.unique(dst)) == len(dst) and not np.isin(dst, src).any()
    src_d = torch.from_numpy(src).to(device)
    dst_d = torch.from_numpy(dst).to(device)
    rng = np.random.default_rng(2)
    same = np.flatnonzero(pairs[:, 0] == pairs[:, 1])
    sample = np.union1d(rng.choice(len(src), size=min(len(src), 6000), replace=False), same)
    m = len(sample)
    s_idx = torch.from_numpy(sample).to(device)
    # source rows are never overwritten (fresh destinations), so they still
    # hold the pre-Reposition values
    host_k = [torch.cat((t[src_d[s_idx]].cpu(), torch.zeros_like(t[src_d[s_idx]].cpu()))) for t in pool.k]
    host_v = [torch.zeros_like(h) for h in host_k]
    cpu_torch.reposition_kv_layers(host_k, host_v, np.arange(m), np.arange(m, 2 * m), pairs[sample], cos_sin.cpu(),
                                   is_neox_style=w.model.is_neox_style)
    for l in range(w.model.n_layers):
        assert torch.equal(pool.v[l][dst_d].view(torch.int16), pool.v[l][src_d].view(torch.int16)), f"V layer {l}"
        got_k = pool.k[l][dst_d[s_idx]].cpu()
        assert torch.equal(got_k.view(torch.int16), host_k[l][m:].view(torch.int16)), f"K layer {l}"


def _edge_workload():
    # raggeds tails, a drop at token 0 (every page copied), a drop on a page
    # boundary, one inside the last page, and a request with no drop at all
    lengths = (37, 160, 100, 64, 33)
    spans = (((0, 5),), ((32, 48), (50, 51)), ((97, 99),), (), ((16, 17),))
    return synth.Workload("paged-edges", synth.TINY, lengths, spans, seed=12, table_positions=200,
                          pool_slots=0, page_size=16, shared_prefix=0)


def test_edge_requests(device):
    w = _edge_workload()
    a = synth.assign_pages(w)
    layouts = synth.compile_layouts(w)
    order = np.arange(w.n_requests) + 1
    table = _table_for(a.birth_rows, 170, device, order)
    got = _run_groups(w, a, layouts, table, order, device)
    torch.cuda.synchronize()
    _check_tables(w, a, layouts, got, table, order)
    # no drop: nothing copied or released, page table unchanged
    assert len(got[3]["copy_source_slots"]) == 0 and len(got[3]["released_pages"]) == 0
    # drop at token 0: every page released, every kept token copied
    assert len(got[0]["released_pages"]) == 3 and len(got[0]["copy_source_slots"]) == 32


def test_row_pointers_and_birth_slots(device):
    w = _edge_workload()
    a = synth.assign_pages(w)
    layouts = synth.compile_layouts(w)
    B = w.n_requests
    rows = [torch.from_numpy(np.concatenate((r, np.full(3, -7, np.int32)))).to(device) for r in a.birth_rows]
    ptrs = torch.tensor([r.data_ptr() for r in rows], dtype=torch.int64, device=device)
    dummy = torch.zeros((1, 1), dtype=torch.int32, device=device)
    inp = tables.pack_paged_inputs(layouts, w.page_size, device)
    out = tables.allocate_paged_outputs(inp, device)
    fresh = torch.from_numpy(np.concatenate(a.fresh_pages).astype(np.int32)).to(device)
    # birth slots given separately; the rows start out holding garbage
    births = torch.from_numpy(np.concatenate(a.birth_rows)).to(device)
    for r in rows:
        r[:-3] = 12345
    tables.compact_pages(inp, dummy, torch.arange(B, dtype=torch.int64, device=device), fresh, out,
                         row_pointers=ptrs, birth_slots=births)
    torch.cuda.synchronize()
    for b, lay in enumerate(layouts):
        want = pg.compact_pages(a.birth_rows[b], lay.keep_mask, lay.birth_positions, lay.positions,
                                a.fresh_pages[b], w.page_size)
        got = rows[b].cpu().numpy()
        np.testing.assert_array_equal(got[:-3], want["terminal_row"])
        assert (got[-3:] == -7).all()


def test_page_one_matches_compact_rows(device):
    case = synth.workload("tiny")
    layouts = synth.compile_layouts(case)
    slots = synth.assign_slots(case, layouts)
    n = case.lengths[0]
    # the row kernel
    inp = tables.pack_compaction_inputs(layouts, device)
    out = tables.allocate_outputs(inp, device)
    t1 = torch.from_numpy(slots.birth_rows[0][None, :].copy()).to(device)
    tables.compact_rows(inp, t1, torch.zeros(1, dtype=torch.int64, device=device),
                        torch.from_numpy(slots.fresh[0]).to(device), out)
    # the page kernel with P = 1 and the same fresh slots as pages
    pin = tables.pack_paged_inputs(layouts, 1, device)
    assert pin.fresh_pages == (len(slots.fresh[0]),)
    pout = tables.allocate_paged_outputs(pin, device)
    t2 = torch.from_numpy(slots.birth_rows[0][None, :].copy()).to(device)
    tables.compact_pages(pin, t2, torch.zeros(1, dtype=torch.int64, device=device),
                         torch.from_numpy(slots.fresh[0]).to(device), pout)
    torch.cuda.synchronize()
    assert torch.equal(t1, t2)
    assert torch.equal(out.copy_src, pout.copy_src)
    assert torch.equal(out.copy_dst, pout.copy_dst)
    assert torch.equal(out.copy_pairs, pout.copy_pairs)
    assert torch.equal(out.retired, pout.released_pages)
    assert torch.equal(out.raw_indices, pout.raw_indices)
    assert torch.equal(out.active_positions, pout.active_positions)
    assert n == t1.shape[1]


@pytest.mark.parametrize("seed", range(10))
def test_random_shared_prefix(device, seed):
    # seeded random batches: page size, prefix, suffixes, drop counts and
    # lengths, and the grouping of requests all vary; a small 2-layer pool
    # checks every copy (K against the oracle's rotation, V bit for bit)
    rng = np.random.default_rng(500 + seed)
    P = int(rng.choice([2, 4, 16, 32, 64]))
    B = int(rng.integers(1, 25))
    prefix = P * int(rng.integers(1, max(2, 640 // P)))
    k_hi = int(rng.integers(0, 7))
    k_lo = int(rng.integers(0, k_hi + 1))
    span_hi = max(1, min(40, (prefix - k_hi) // max(k_hi, 1) - 1))
    suffix_hi = int(rng.integers(0, 200))
    w = synth.shared_prefix_workload(f"paged-random-{seed}", synth.TINY, B, prefix, 0, suffix_hi, k_lo, k_hi,
                                     1, span_hi, P, seed=seed)
    if rng.random() < 0.5:
        split = None
    else:
        perm = rng.permutation(B)
        cuts = np.sort(rng.choice(np.arange(1, B), size=min(B - 1, int(rng.integers(0, 4))), replace=False))
        split = [list(g) for g in np.split(perm, cuts)]
    a = synth.assign_pages(w, split)
    layouts = synth.compile_layouts(w)
    print(f"paged random {seed}: P={P} B={B} prefix={prefix} groups={len(a.groups)} pages={a.pool_pages}",
          flush=True)
    pool = synth.make_pool(w.model, a.pool_pages * P, device, seed=seed)
    cos_sin = synth.rope_table(w, device)
    k_before = [t.clone() for t in pool.k]
    v_before = [t.clone() for t in pool.v]
    order = rng.permutation(B + 3)[:B]
    table = _table_for(a.birth_rows, max(w.lengths) + 5, device, order)
    got = _run_groups(w, a, layouts, table, order, device, pool, cos_sin)
    torch.cuda.synchronize()
    _check_tables(w, a, layouts, got, table, order)

    src = np.concatenate([got[b]["copy_source_slots"] for b in range(B)]).astype(np.int64)
    dst = np.concatenate([got[b]["copy_destination_slots"] for b in range(B)]).astype(np.int64)
    pairs = np.concatenate([got[b]["copy_position_pairs"] for b in range(B)]).reshape(-1, 2)
    assert len(np.unique(dst)) == len(dst)
    untouched = np.ones(a.pool_pages * P, dtype=bool)
    untouched[dst] = False
    table_np = to_storage(cos_sin)
    for l in range(w.model.n_layers):
        k0, v0 = to_storage(k_before[l]), to_storage(v_before[l])
        k1, v1 = to_storage(pool.k[l]), to_storage(pool.v[l])
        np.testing.assert_array_equal(v1[dst], v0[src], err_msg=f"V of layer {l}")
        np.testing.assert_array_equal(k1[untouched], k0[untouched], err_msg=f"K of layer {l}")
        np.testing.assert_array_equal(v1[untouched], v0[untouched], err_msg=f"V of layer {l}")
        m = len(src)
        kk = [np.concatenate((k0[src], np.zeros((m,) + k0.shape[1:], np.uint16)))]
        vv = [np.zeros_like(kk[0])]
        rp.reposition_kv_layers(kk, vv, np.arange(m), np.arange(m, 2 * m), pairs, table_np, dtype="bf16")
        assert storage_equal(k1[dst], kk[0][m:]), f"K of layer {l}"
