"""The whole GPU step (compaction + Reposition + decode indices) captured in
a HIP graph: every replay must reproduce the eager results."""

import numpy as np
import pytest
import torch

from akv_amd import ops, page_table, synth, tables

from harness import attention_metadata, plain_segments, prefill_forward

pytestmark = pytest.mark.gpu


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
    kept = int(lay.keep_mask.sum())
    # registry row 1: the request's final active versions, as compacted
    registry = torch.zeros((2, 6), dtype=torch.int64)
    registry[1] = torch.tensor([out.raw_indices.data_ptr(), out.active_positions.data_ptr(), n, kept,
                                lay.next_position, 0], dtype=torch.int64)
    registry = registry.to(device)
    seq = torch.tensor([kept + 1], dtype=torch.int64, device=device)
    indptr = torch.empty(2, dtype=torch.int32, device=device)
    kv = torch.empty(kept + 1, dtype=torch.int32, device=device)
    torch.cuda.synchronize()

    def step():
        tables.compact_rows(inputs, table, rows, fresh, out, generated=gen, birth_slots=birth)
        ops.reposition_kv_layers_gated(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src,
                                       out.copy_dst, out.copy_pairs, rope, status=out.status)
        page_table.build_indptr(seq, indptr)
        page_table.context_decode_indices(registry, table, rows, seq, indptr, kv, status=out.status)

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
        assert int(out.status.item()) == 0, f"replay {replay}"
        for t, x in zip(pool.k + pool.v, want_kv):
            assert torch.equal(t[dst].view(torch.int16), x.view(torch.int16)), f"replay {replay}"
    assert np.array_equal(kv.cpu().numpy(), out.kv_indices.cpu().numpy())


def test_graph_replays_attention_consumers(device):
    """Decode attention (with its workspace) and the prefill attention over
    fixed metadata captured in one graph: replays equal the eager outputs."""
    from akv_amd import attention

    g = torch.Generator(device=device).manual_seed(21)
    hq, hkv, d = 64, 8, 64
    slots = 6000
    k = torch.randn((slots, hkv, d), generator=g, device=device).to(torch.bfloat16)
    v = torch.randn((slots, hkv, d), generator=g, device=device).to(torch.bfloat16)
    rng = np.random.default_rng(21)
    lengths = [300, 1, 2000, 57]
    indptr = torch.tensor(np.concatenate(([0], np.cumsum(lengths))), dtype=torch.int32, device=device)
    idx = torch.from_numpy(rng.integers(1, slots, size=sum(lengths)).astype(np.int32)).to(device)
    q = torch.randn((len(lengths), hq, d), generator=g, device=device).to(torch.bfloat16)
    sinks = torch.randn(hq, generator=g, device=device)
    o_dec = torch.empty_like(q)
    ws = torch.empty(attention.workspace_bytes(len(lengths), hkv, d, max(lengths)) // 4 + 1, dtype=torch.float32,
                     device=device)
    requests = [plain_segments(500, 77), plain_segments(0, 30)]
    occ = torch.from_numpy(rng.permutation(np.arange(1, slots))[: sum(r.occurrences for r in requests)]
                           .astype(np.int64)).to(device)
    meta = attention_metadata(requests, occ)
    nq = meta.query_count
    qe = torch.randn((nq, hq, d), generator=g, device=device).to(torch.bfloat16)
    ke = torch.randn((nq, hkv, d), generator=g, device=device).to(torch.bfloat16)
    ve = torch.randn((nq, hkv, d), generator=g, device=device).to(torch.bfloat16)
    o_pre = torch.empty_like(qe)
    torch.cuda.synchronize()

    def step():
        attention.decode_attention(q, k, v, indptr, idx, o_dec, scale=0.125, max_len=max(lengths), sinks=sinks,
                                   workspace=ws)
        prefill_forward(meta, qe, ke, ve, o_pre, k, v, sm_scale=0.125, sliding_window_size=64, sinks=sinks)

    step()
    torch.cuda.synchronize()
    want = [o_dec.clone(), o_pre.clone()]
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step()
    for replay in range(4):
        o_dec.fill_(3.0)
        o_pre.fill_(3.0)
        ws.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_dec.view(torch.int16), want[0].view(torch.int16)), f"replay {replay}"
        assert torch.equal(o_pre.view(torch.int16), want[1].view(torch.int16)), f"replay {replay}"
