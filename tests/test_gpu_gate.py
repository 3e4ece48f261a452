"""The compaction's device status word as its consumers' gate, and the
one-pass compaction's fallback rebuild.

The lists go from ``akv_compact_rows`` to the Reposition, the decode index
and attention kernels and the row copy on one stream with no host read:
each consumer reads the status word on the device and, when it marks the
lists unusable, touches no K/V row and writes nothing.  The lists given
here always hold valid, in-range slots (a real compaction's), so even a
broken gate could not make a kernel read out of bounds; a closed gate is
seen as buffers left bit-for-bit unchanged.

The one-pass compaction's tiles meet at an in-kernel barrier with bounded
waits; a tile whose wait runs out skips its outputs and the finishing
launch rebuilds them.  The test forces that path from the host with a
stale arrival counter in the workspace (every wait still ends at its
bound), then checks every output against the oracle and that the next call
on the same workspace takes the fast path again.
"""

import time

import numpy as np
import pytest
import torch

from akv_amd import _lib, attention, ops, page_table, synth, tables, transfer
from test_gpu_compact import _check, _path, _setup

pytestmark = pytest.mark.gpu

# int32 words between the arrival counters of two groups in the workspace
# (one 128-byte line each, at the start of the workspace)
ARRIVAL_STRIDE = 32


def _compacted_tiny(device):
    w = synth.workload("tiny")
    layouts = synth.compile_layouts(w)
    slots, inputs, table, req_rows, fresh, _, _, _ = _setup(device, w, layouts, generated=[1])
    # the generated token's entry must be a slot of the pool (the decode
    # attention below reads it)
    used = np.concatenate(slots.birth_rows + slots.fresh)
    table[int(req_rows[0]), w.lengths[0]] = int(np.setdiff1d(np.arange(1, w.pool_slots), used)[0])
    out = tables.allocate_outputs(inputs, device, generated_total=1)
    tables.compact_rows(inputs, table, req_rows, fresh, out, generated=torch.ones(1, dtype=torch.int32,
                                                                                    device=device))
    torch.cuda.synchronize()
    assert tables.check_status(out) == 0
    assert int(out.kv_indices.max()) < w.pool_slots and int(out.kv_indices.min()) > 0
    return w, layouts, inputs, table, req_rows, out


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


@pytest.mark.parametrize("code", [_lib.AKV_STATUS_SIZES, _lib.AKV_STATUS_INCOMPLETE, 3, 7])
def test_closed_gate_blocks_every_consumer(device, code):
    w, layouts, inputs, table, req_rows, out = _compacted_tiny(device)
    m = w.model
    pool = synth.make_pool(m, w.pool_slots, device, seed=3, generate_on_device=False)
    rope = synth.rope_table(w, device)
    before = [t.clone() for t in pool.k + pool.v]
    out.status.fill_(code)
    print(f"gate closed with status {code}", flush=True)

    ops.reposition_kv_layers_gated(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src, out.copy_dst,
                                   out.copy_pairs, rope, status=out.status)
    transfer.copy_kv_rows(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.k_ptrs, pool.v_ptrs, pool.k[0],
                          inputs.moved_total, src_slots=out.copy_src, dst_slots=out.copy_dst, status=out.status)
    n = w.lengths[0]
    registry = torch.zeros((table.shape[0], 6), dtype=torch.int64)
    row = int(req_rows[0])
    registry[row] = torch.tensor([out.raw_indices.data_ptr(), out.active_positions.data_ptr(), n,
                                  inputs.kept[0], layouts[0].next_position, 0])
    registry = registry.to(device)
    seq = torch.tensor([inputs.kept[0] + 1], dtype=torch.int64, device=device)
    indptr = torch.tensor([0, inputs.kept[0] + 1], dtype=torch.int32, device=device)
    idx = torch.full((inputs.kept[0] + 1,), -7, dtype=torch.int32, device=device)
    page_table.context_decode_indices(registry, table, req_rows, seq, indptr, idx, status=out.status)
    q = torch.randn((1, 2 * m.n_heads, m.head_dim), device=device).to(torch.bfloat16)
    o = torch.full(q.shape, float("nan"), dtype=torch.float32, device=device)
    attention.decode_attention(q, pool.k[0], pool.v[0], out.kv_indptr, out.kv_indices, o, scale=0.125,
                               max_len=inputs.kept[0] + 1, status=out.status)
    torch.cuda.synchronize()
    for t, b in zip(pool.k + pool.v, before):
        assert torch.equal(_bits(t), _bits(b)), "a gated kernel wrote K/V rows"
    assert bool((idx == -7).all()), "gated decode indices wrote output"
    assert bool(torch.isnan(o).all()), "gated decode attention wrote output"

    # an open gate (0, or the informational rebuilt bit) lets every consumer run
    for open_code in (0, _lib.AKV_STATUS_REBUILT):
        out.status.fill_(open_code)
        ops.reposition_kv_layers_gated(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src,
                                       out.copy_dst, out.copy_pairs, rope, status=out.status)
        page_table.context_decode_indices(registry, table, req_rows, seq, indptr, idx, status=out.status)
        attention.decode_attention(q, pool.k[0], pool.v[0], out.kv_indptr, out.kv_indices, o, scale=0.125,
                                   max_len=inputs.kept[0] + 1, status=out.status)
        torch.cuda.synchronize()
        assert torch.equal(idx, out.kv_indices)
        assert bool(torch.isfinite(o).all())
    dst = out.copy_dst.long()
    got = [t[dst].clone() for t in pool.k + pool.v]
    for t, b in zip(pool.k + pool.v, before):
        t.copy_(b)
    ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src, out.copy_dst,
                             out.copy_pairs, rope)
    torch.cuda.synchronize()
    for t, g in zip(pool.k + pool.v, got):
        assert torch.equal(_bits(t[dst]), _bits(g))


def test_size_mismatch_status_gates_the_reposition(device):
    """A compaction given one fresh slot too few reports AKV_STATUS_SIZES; the
    gated Reposition then leaves the pool untouched.  The lists are pre-filled
    with valid slots, so entries the compaction leaves unwritten are valid
    too."""
    w = synth.workload("tiny")
    layouts = synth.compile_layouts(w)
    slots, inputs, table, req_rows, fresh, _, _, _ = _setup(device, w, layouts)
    out = tables.allocate_outputs(inputs, device)
    for t in (out.copy_src, out.copy_dst):
        t.fill_(1)
    out.copy_pairs.fill_(0)
    inputs_bad = tables.CompactionInputs(**{**inputs.__dict__, "moved": (inputs.moved[0] - 1,)})
    out.copy_src, out.copy_dst, out.copy_pairs = out.copy_src[:-1], out.copy_dst[:-1], out.copy_pairs[:-1]
    tables.compact_rows(inputs_bad, table, req_rows, fresh[:-1], out)
    pool = synth.make_pool(w.model, w.pool_slots, device, seed=4, generate_on_device=False)
    rope = synth.rope_table(w, device)
    before = [t.clone() for t in pool.k + pool.v]
    ops.reposition_kv_layers_gated(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src, out.copy_dst,
                                   out.copy_pairs, rope, status=out.status)
    torch.cuda.synchronize()
    assert int(out.status.item()) & _lib.AKV_STATUS_SIZES
    with pytest.raises(RuntimeError, match="does not match"):
        tables.check_status(out)
    for t, b in zip(pool.k + pool.v, before):
        assert torch.equal(_bits(t), _bits(b))


@pytest.mark.parametrize("stale_groups", [(0,), (1,)], ids=["every-group", "second-group"])
def test_fallback_rebuilds_tiles_that_stopped_waiting(device, stale_groups):
    """The 32k request on the one-pass path (128 tiles, 2 groups).  A stale
    arrival counter (a value no arrival reaches) leaves its group without a
    releaser: the group's tiles wait out their bound and withdraw (and with
    group 0 stale, group 1's look-back runs out too).  The finishing launch
    rebuilds exactly those tiles; every output matches the oracle, the
    status reads AKV_STATUS_REBUILT, and the next call on the same workspace
    takes the fast path (status 0) with the same outputs."""
    lib = _lib.load()
    w = synth.workload("gpt-oss-32k")
    assert _path(lib, 1, sum(w.lengths)) == (1, 256)
    layouts = synth.compile_layouts(w)
    slots, inputs, table, req_rows, fresh, _, _, tails = _setup(device, w, layouts, generated=[1])
    birth = table[int(req_rows[0])].clone()
    out = tables.allocate_outputs(inputs, device, generated_total=1)
    gen = torch.ones(1, dtype=torch.int32, device=device)
    words = out.workspace.view(torch.int32)
    for k in stale_groups:
        words[k * ARRIVAL_STRIDE] = 1000
    print(f"stale arrival counter in groups {stale_groups}: expect tens of ms of bounded waiting", flush=True)
    for call in range(2):
        table[int(req_rows[0])] = birth
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tables.compact_rows(inputs, table, req_rows, fresh, out, generated=gen)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3
        status = int(out.status.item())
        print(f"call {call}: status {status}, {ms:.2f} ms", flush=True)
        assert status == (_lib.AKV_STATUS_REBUILT if call == 0 else 0)
        out.status.zero_()
        rows_after = [table[r].cpu().numpy() for r in req_rows.cpu().numpy()]
        _check(w, layouts, slots, out, rows_after, tails, [1])
    # the finishing launch reset the arrival counters
    assert int(words[: 32 * ARRIVAL_STRIDE : ARRIVAL_STRIDE].abs().sum()) == 0
