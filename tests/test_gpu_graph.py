"""The whole GPU step (compaction + Reposition + decode indices) captured in
a HIP graph: every replay must reproduce the eager results."""

import numpy as np
import pytest
import torch

from akv_amd import ops, page_table, synth, tables

pytestmark = pytest.mark.gpu


class _T:
    page_size, defer_read_translate, is_translating = 1, False, False

    def __init__(self, table):
        self.req_to_token = table


def test_graph_replays_match_eager(device):
    w = synth.workload("tiny")
    layouts = synth.compile_layouts(w)
    lay = layouts[0]
    slots = synth.assign_slots(w, layouts)
    n = w.lengths[0]
    inputs = tables.pack_compaction_inputs(layouts, device)
    out = tables.allocate_outputs(inputs, device, generated_total=1)
    table = torch.full((2, n + 4), -1, dtype=torch.int32, device=device)
    table[1, n] = 99
    birth = torch.from_numpy(slots.birth_rows[0]).to(device)
    fresh = torch.from_numpy(slots.fresh[0]).to(device)
    rows = torch.tensor([1], dtype=torch.int64, device=device)
    gen = torch.ones(1, dtype=torch.int32, device=device)
    pool = synth.make_pool(w.model, w.pool_slots, device, seed=3, generate_on_device=False)
    rope = synth.rope_table(w, device)
    registry = page_table.ContextDecodeRegistry(_T(table), pool=None)
    kept = int(lay.keep_mask.sum())
    registry.rows[1] = torch.tensor([out.raw_indices.data_ptr(), out.active_positions.data_ptr(), n, kept,
                                     lay.next_position, 0], dtype=torch.int64)
    seq = torch.tensor([kept + 1], dtype=torch.int64, device=device)
    indptr = torch.empty(2, dtype=torch.int32, device=device)
    kv = torch.empty(kept + 1, dtype=torch.int32, device=device)
    torch.cuda.synchronize()

    def step():
        tables.compact_rows(inputs, table, rows, fresh, out, generated=gen, birth_slots=birth)
        ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src, out.copy_dst,
                                 out.copy_pairs, rope)
        page_table.build_indptr(seq, indptr)
        registry.fill(rows, seq, indptr, kv)

    dst = fresh.long()
    step()
    torch.cuda.synchronize()
    want = [t.clone() for t in (table, out.retired, out.copy_src, out.copy_pairs, out.kv_indices, kv, indptr)]
    want_kv = [t[dst].clone() for t in pool.k + pool.v]

    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()  # warm the side stream once, outside capture
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step()
    for replay in range(4):
        # eager corruption of every output between replays (the prompt part
        # of the request row; its generated column is an input)
        table[1, :n].fill_(-5)
        for t in (out.retired, out.copy_src, out.copy_pairs, out.kv_indices, kv, indptr):
            t.fill_(-7)
        for t in pool.k + pool.v:
            t[dst] = 0
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [table, out.retired, out.copy_src, out.copy_pairs, out.kv_indices, kv, indptr]
        for g, x in zip(got, want):
            assert torch.equal(g, x), f"replay {replay}"
        for t, x in zip(pool.k + pool.v, want_kv):
            assert torch.equal(t[dst].view(torch.int16), x.view(torch.int16)), f"replay {replay}"
    assert np.array_equal(kv.cpu().numpy(), out.kv_indices.cpu().numpy())
