"""GPU parity of the decode-metadata kernels and the registry interface."""

import numpy as np
import pytest
import torch

from akv_amd import page_table as pt
from akv_amd import synth, tables
from oracle import decode as dec
from oracle import occurrence as occ

pytestmark = pytest.mark.gpu


class _Translator:
    page_size = 1
    defer_read_translate = False
    is_translating = False

    def __init__(self, req_to_token):
        self.req_to_token = req_to_token


class _Req:
    def __init__(self, layout, row):
        self.context_program = None if layout is None else type("P", (), {"layout": layout})()
        self.context_decode_layout = None
        self.kv = type("K", (), {"req_pool_idx": row})()


def _batch(device, seed=0, batch=24):
    rng = np.random.default_rng(seed)
    width = 3000
    table = np.full((batch + 4, width), -3, dtype=np.int32)
    reqs, raw_lengths, expect = [], [], []
    for b in range(batch):
        row = b + 2
        n = int(rng.integers(20, 2500))
        gen = int(rng.integers(1, 6))
        slots = rng.integers(1, 10**7, size=n + gen).astype(np.int32)
        if rng.random() < 0.25:
            table[row, : n + gen] = slots
            reqs.append(_Req(None, row))
            raw_lengths.append(n + gen)
            expect.append((None, slots.copy(), gen))
            continue
        k = int(rng.integers(1, 4))
        cuts = np.sort(rng.choice(np.arange(n), size=2 * k, replace=False))
        spans = tuple((int(cuts[2 * j]), int(cuts[2 * j + 1])) for j in range(k))
        lay = synth.compile_context_layout(**synth.request_events(n, spans))
        moved = lay.keep_mask.numpy() & (lay.birth_positions.numpy() != lay.positions.numpy())
        cf = occ.closed_form(slots[:n], lay.keep_mask.numpy(), lay.birth_positions.numpy(), lay.positions.numpy(),
                             rng.integers(1, 10**7, size=int(moved.sum())))
        table[row, :n] = cf["terminal_row"]
        table[row, n : n + gen] = slots[n:]
        reqs.append(_Req(lay, row))
        raw_lengths.append(n + gen)
        expect.append((lay, np.concatenate((cf["active_slots"], slots[n:])), gen))
    return torch.from_numpy(table).to(device), reqs, raw_lengths, expect


def test_registry_fill_matches_compacted_rows(device):
    table, reqs, raw_lengths, expect = _batch(device)
    registry = pt.ContextDecodeRegistry(_Translator(table), pool=None)
    row_ids = torch.tensor([r.kv.req_pool_idx for r in reqs], dtype=torch.int64, device=device)
    lengths, _, positions, refs = registry.bind_batch(reqs, raw_lengths, row_ids)
    seq = lengths.to(device)
    for out_dtype in (torch.int32, torch.int64):
        indptr = torch.empty(len(reqs) + 1, dtype=torch.int32, device=device)
        pt.build_indptr(seq, indptr)
        out = torch.full((int(lengths.sum()),), -9, dtype=out_dtype, device=device)
        registry.fill(row_ids, seq, indptr, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ip = indptr.cpu().numpy()
        np.testing.assert_array_equal(ip, dec.kv_indptr(lengths.numpy()))
        for b, (_, want, _) in enumerate(expect):
            np.testing.assert_array_equal(got[ip[b] : ip[b + 1]], want)
    # query positions: next_position + generated - 1
    for b, (lay, _, gen) in enumerate(expect):
        if lay is not None:
            assert int(positions[b]) == lay.next_position + gen - 1


@pytest.mark.parametrize("window", [0, 1, 7, 128, 5000])
def test_fill_window_and_table_match_oracle(device, window):
    table, reqs, raw_lengths, expect = _batch(device, seed=1)
    registry = pt.ContextDecodeRegistry(_Translator(table), pool=None)
    row_ids = torch.tensor([r.kv.req_pool_idx for r in reqs], dtype=torch.int64, device=device)
    lengths, _, _, refs = registry.bind_batch(reqs, raw_lengths, row_ids)
    seq = lengths.to(device)
    reg_np = registry.rows.cpu().numpy()
    memory = {}
    for r in reqs:
        lay = r.context_decode_layout
        if lay is not None:
            memory[lay.device_indices.data_ptr()] = lay.raw_indices
            memory[lay.device_positions.data_ptr()] = lay.positions
    want_len = dec.window_lengths(reg_np, row_ids.cpu().numpy(), lengths.numpy(), window, memory=memory)
    indptr_buf = torch.zeros(len(reqs) + 8, dtype=torch.int32, device=device)
    out = torch.zeros(int(want_len.sum()) + 5, dtype=torch.int64, device=device)
    indptr, _, got_len, starts = registry.fill_window(row_ids, seq, indptr_buf, window, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got_len.cpu().numpy(), want_len)
    ip = indptr.cpu().numpy()
    np.testing.assert_array_equal(ip, dec.kv_indptr(want_len))
    for b, (_, full, _) in enumerate(expect):
        s = int(lengths[b]) - int(want_len[b])
        np.testing.assert_array_equal(out.cpu().numpy()[ip[b] : ip[b + 1]], full[s:])
    # dense page-one table form (FA3 style)
    dense = torch.full((len(reqs), 3000), -1, dtype=torch.int32, device=device)
    got = registry.fill_table(row_ids, seq, dense, window=window)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want_len)
    d = dense.cpu().numpy()
    for b, (_, full, _) in enumerate(expect):
        s = int(lengths[b]) - int(want_len[b])
        np.testing.assert_array_equal(d[b, : want_len[b]], full[s:])


def test_mapping_translation_and_row_slots(device):
    table, reqs, raw_lengths, expect = _batch(device, seed=2, batch=6)
    mapping = (torch.arange(10**7, dtype=torch.int64) * 5 + 3).to(device)
    t = _Translator(table)
    t.is_translating = True
    t._full_v2p_table = mapping
    t._full_page_multiplier = 2
    registry = pt.ContextDecodeRegistry(t, pool=None)
    row_ids = torch.tensor([r.kv.req_pool_idx for r in reqs], dtype=torch.int32, device=device)
    lengths, _, _, _ = registry.bind_batch(reqs, raw_lengths, row_ids)
    seq = lengths.to(device)
    indptr = torch.empty(len(reqs) + 1, dtype=torch.int64, device=device)
    pt.build_indptr(seq, indptr)
    out = torch.zeros(int(lengths.sum()), dtype=torch.int64, device=device)
    registry.fill(row_ids, seq, indptr, out)
    torch.cuda.synchronize()
    ip = indptr.cpu().numpy()
    for b, (_, want, _) in enumerate(expect):
        np.testing.assert_array_equal(out.cpu().numpy()[ip[b] : ip[b + 1]], (want.astype(np.int64) * 5 + 3) * 2)
    # side-row scatter
    rows = [torch.zeros(16, dtype=torch.int32, device=device) for _ in range(3)]
    pointers = torch.tensor([r.data_ptr() for r in rows], dtype=torch.int64, device=device)
    pt.write_row_slots(pointers, torch.tensor([0, 2, 2, 1], device=device),
                       torch.tensor([1, 0, 15, 7], dtype=torch.int32, device=device),
                       torch.tensor([11, 22, 33, 44], dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert rows[0].cpu().tolist()[1] == 11 and rows[1].cpu().tolist()[7] == 44
    assert rows[2].cpu().tolist()[0] == 22 and rows[2].cpu().tolist()[15] == 33


def test_indptr_and_last_page(device):
    rng = np.random.default_rng(3)
    for batch in (1, 7, 64, 1500):
        lengths = rng.integers(0, 70000, size=batch)
        seq = torch.from_numpy(lengths).to(device)
        indptr = torch.empty(batch + 1, dtype=torch.int64, device=device)
        last = torch.empty(batch, dtype=torch.int32, device=device)
        pt.build_indptr(seq, indptr, last_page_len=last, page_size=16)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(indptr.cpu().numpy(), dec.kv_indptr(lengths))
        np.testing.assert_array_equal(last.cpu().numpy(), dec.last_page_lengths(lengths, 16))


def test_pipeline_compaction_feeds_registry(device):
    """compact_rows outputs bind directly as registry rows (no host round trip)."""
    w = synth.workload("ragged-64")
    layouts = synth.compile_layouts(w)
    slots = synth.assign_slots(w, layouts)
    inputs = tables.pack_compaction_inputs(layouts, device)
    width = max(w.lengths) + 4
    table = torch.full((w.n_requests, width), -1, dtype=torch.int32)
    for b in range(w.n_requests):
        table[b, : w.lengths[b]] = torch.from_numpy(slots.birth_rows[b])
        table[b, w.lengths[b]] = 7  # one generated token's slot
    table = table.to(device)
    fresh = torch.from_numpy(np.concatenate(slots.fresh)).to(device)
    out = tables.allocate_outputs(inputs, device, generated_total=w.n_requests)
    gen = torch.ones(w.n_requests, dtype=torch.int32, device=device)
    row_ids = torch.arange(w.n_requests, dtype=torch.int64, device=device)
    tables.compact_rows(inputs, table, row_ids, fresh, out, generated=gen)
    registry = pt.ContextDecodeRegistry(_Translator(table), pool=None)
    kept_off = np.concatenate(([0], np.cumsum(inputs.kept)))
    rows = []
    for b, lay in enumerate(layouts):
        raw_ptr = out.raw_indices.data_ptr() + 4 * int(kept_off[b])
        pos_ptr = out.active_positions.data_ptr() + 4 * int(kept_off[b])
        rows.append((raw_ptr, pos_ptr, w.lengths[b], inputs.kept[b], lay.next_position, 0))
    registry.rows[row_ids] = torch.tensor(rows, dtype=torch.int64).to(device)
    seq = torch.tensor([k + 1 for k in inputs.kept], dtype=torch.int64, device=device)
    indptr = torch.empty(w.n_requests + 1, dtype=torch.int32, device=device)
    pt.build_indptr(seq, indptr)
    kv = torch.empty(int(seq.sum()), dtype=torch.int32, device=device)
    registry.fill(row_ids, seq, indptr, kv)
    torch.cuda.synchronize()
    assert torch.equal(kv, out.kv_indices)
    assert torch.equal(indptr, out.kv_indptr)
