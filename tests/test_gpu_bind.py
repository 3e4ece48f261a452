"""GPU parity of the occurrence binding of multi-stage whole-prompt forwards
against the oracle's restated planner (plan_final_forward +
advance_final_forward), and the prefill attention reading the bound
occurrence slots after the Reposition of the copies."""

import numpy as np
import pytest
import torch

from akv_amd import occurrence as ow
from akv_amd import ops, plan
from akv_amd.rope import make_table
from oracle import attention as oat
from oracle import events as ev
from oracle import occurrence as occ

from harness import attention_metadata, prefill_forward, window_segments
from test_occurrence_window import _program, _torch_layout

pytestmark = pytest.mark.gpu


def _request(rng, n):
    events, visible = _program(rng, n)
    ref = ev.compile_context_layout(*(np.asarray(events[k]) for k in events))
    lay = _torch_layout(events)
    vis = torch.from_numpy(np.minimum(visible, 2**31 - 1).astype(np.int32))
    window = ow.compile_occurrence_window(lay, vis, lay.positions, query_start=0, query_end=n)
    return ref, lay, visible, window


def _bind_batch(device, reqs, rng):
    windows = [r[3] for r in reqs]
    keeps = [np.asarray(r[1].keep_mask, dtype=bool) for r in reqs]
    inp = ow.pack_final_forward(windows, keeps, device)
    out = ow.allocate_final_forward_outputs(inp, device)
    total = sum(inp.n_tokens) + sum(inp.extra)
    slots = rng.permutation(np.arange(1, 3 * total + 10)).astype(np.int32)
    birth = slots[: sum(inp.n_tokens)]
    fresh = slots[sum(inp.n_tokens) : total]
    B = len(reqs)
    order = rng.permutation(B + 2)[:B]
    table = torch.full((B + 2, max(inp.n_tokens) + 3), -7, dtype=torch.int32, device=device)
    ow.bind_final_forward(inp, table, torch.from_numpy(order.astype(np.int64)).to(device),
                          torch.from_numpy(birth).to(device), torch.from_numpy(fresh).to(device), out)
    torch.cuda.synchronize()
    return inp, out, birth, fresh, table, order


def _check(reqs, inp, out, birth, fresh, table, order):
    bases = inp.bases.cpu().numpy()
    occ_slots = out.occurrence_slots.cpu().numpy()
    src, dst, pairs = out.copy_src.cpu().numpy(), out.copy_dst.cpu().numpy(), out.copy_pairs.cpu().numpy()
    retired = out.retired.cpu().numpy()
    tab = table.cpu().numpy()
    for b, (ref, lay, visible, window) in enumerate(reqs):
        n = inp.n_tokens[b]
        p = occ.plan_final_forward(ref, visible)
        want = occ.advance_final_forward(ref, p, birth[bases[1, b] : bases[1, b + 1]],
                                         fresh[bases[2, b] : bases[2, b + 1]])
        c = slice(bases[2, b], bases[2, b + 1])
        np.testing.assert_array_equal(src[c], want["copy_source_slots"], err_msg=f"request {b}")
        np.testing.assert_array_equal(dst[c], want["copy_destination_slots"])
        np.testing.assert_array_equal(pairs[c], want["copy_position_pairs"])
        np.testing.assert_array_equal(retired[bases[3, b] : bases[3, b + 1]], want["retired_slots"])
        np.testing.assert_array_equal(tab[order[b], :n], want["terminal_row"])
        assert (tab[order[b], n:] == -7).all()
        got_occ = occ_slots[bases[0, b] : bases[0, b + 1]]
        required = p["source_rows"] >= 0
        required[p["allocated"]] = True
        np.testing.assert_array_equal(got_occ[required], want["occurrence_slots"][required])
        assert (got_occ[~required] == -1).all()


def test_batched_multi_stage_programs(device):
    rng = np.random.default_rng(11)
    reqs = [_request(rng, int(rng.integers(8, 400))) for _ in range(40)]
    assert sum(r[3].first_final_occurrence > len(r[3].terminal_occurrences) for r in reqs) > 20
    _check(reqs, *_bind_batch(device, reqs, rng))


@pytest.mark.parametrize("seed", range(8))
def test_random_batches(device, seed):
    # seeded random batches of random multi-stage programs: 1-60 requests of
    # 8-3000 tokens (programs need a few tokens), a few long ones among many short
    rng = np.random.default_rng(1100 + seed)
    B = int(rng.integers(1, 61))
    lengths = np.where(rng.random(B) < 0.8, rng.integers(8, 300, size=B), rng.integers(300, 3001, size=B))
    print(f"bind random {seed}: B={B} tokens={int(lengths.sum())}", flush=True)
    reqs = [_request(rng, int(n)) for n in lengths]
    _check(reqs, *_bind_batch(device, reqs, rng))


def test_long_request_spans_many_tiles(device):
    rng = np.random.default_rng(12)
    reqs = [_request(rng, 20000), _request(rng, 12), _request(rng, 3000)]
    _check(reqs, *_bind_batch(device, reqs, rng))


def test_prefill_reads_bound_occurrences_after_reposition(device):
    """Window -> device binding -> Reposition of the copies -> context
    attention over the window's segments, against the oracle attention over
    the same pool rows (K/V gathered at the oracle's occurrence slots)."""
    rng = np.random.default_rng(13)
    ref, lay, visible, window = _request(rng, 600)
    reqs = [(ref, lay, visible, window)]
    inp, out, birth, fresh, table, order = _bind_batch(device, reqs, rng)
    _check(reqs, inp, out, birth, fresh, table, order)
    hq, hkv, d = 8, 1, 64
    slots = int(max(birth.max(), fresh.max() if len(fresh) else 0)) + 1
    g = torch.Generator().manual_seed(5)
    k_pool = torch.randn((slots, hkv, d), generator=g).to(torch.bfloat16).to(device)
    v_pool = torch.randn((slots, hkv, d), generator=g).to(torch.bfloat16).to(device)
    n = len(window.terminal_occurrences)
    # the extend's own K/V rows are the queries' birth rows of the pool
    births = torch.from_numpy(birth.astype(np.int64)).to(device)
    k_ext, v_ext = k_pool[births].contiguous(), v_pool[births].contiguous()
    table_rope = make_table("plain", d, 4096, base=10000.0, device=device)
    ptr_k = torch.tensor([k_pool.data_ptr()], dtype=torch.uint64, device=device)
    ptr_v = torch.tensor([v_pool.data_ptr()], dtype=torch.uint64, device=device)
    ops.reposition_kv_layers(ptr_k, ptr_v, k_pool, v_pool, out.copy_src, out.copy_dst, out.copy_pairs, table_rope)
    meta = attention_metadata([window_segments(window)], out.occurrence_slots.long())
    q = torch.randn((n, hq, d), generator=g).to(torch.bfloat16).to(device)
    o = torch.empty_like(q)
    prefill_forward(meta, q, k_ext, v_ext, o, k_pool, v_pool, sliding_window_size=-1)
    torch.cuda.synchronize()
    c = meta.cpu
    want_slots = occ.advance_final_forward(ref, occ.plan_final_forward(ref, visible), birth, fresh)["occurrence_slots"]
    f32 = lambda t: t.float().cpu().numpy()
    want = oat.context_attention(f32(q), f32(k_ext), f32(v_ext), f32(k_pool), f32(v_pool), c.qo_indptr, c.kv_indptr,
                                 want_slots[c.occurrences], d ** -0.5, q_positions=c.query_positions,
                                 kv_positions=c.kv_positions)
    assert np.abs(f32(o) - want).max() <= 2e-2
