"""GPU parity of the decode-metadata kernels (read indices, window lengths,
indptr rebuild, side-row scatter), driven the way a decode registry drives
them: one int64 row per request pointing at its final active versions."""

import numpy as np
import pytest
import torch

from akv_amd import page_table as pt
from akv_amd import synth, tables
from oracle import decode as dec
from oracle import occurrence as occ

from harness import DecodeRows, dense_indices, window_indices

pytestmark = pytest.mark.gpu


def _batch(device, seed=0, batch=24):
    """Requests in table rows 2 .. batch+1: a quarter ordinary, the rest after
    a final forward (terminal row), each with a few generated tokens."""
    rng = np.random.default_rng(seed)
    width = 3000
    table = np.full((batch + 4, width), -3, dtype=np.int32)
    entries, seq, expect = [], [], []
    for b in range(batch):
        row = b + 2
        n = int(rng.integers(20, 2500))
        gen = int(rng.integers(1, 6))
        slots = rng.integers(1, 10**7, size=n + gen).astype(np.int32)
        if rng.random() < 0.25:
            table[row, : n + gen] = slots
            entries.append((row, None))
            seq.append(n + gen)
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
        entries.append((row, lay))
        seq.append(int(lay.keep_mask.sum()) + gen)
        expect.append((lay, np.concatenate((cf["active_slots"], slots[n:])), gen))
    table = torch.from_numpy(table).to(device)
    reg = DecodeRows.from_layouts(batch + 4, entries, device)
    row_ids = torch.tensor([r for r, _ in entries], dtype=torch.int64, device=device)
    return table, reg, row_ids, np.asarray(seq, dtype=np.int64), expect


def test_read_indices_match_compacted_rows(device):
    table, reg, row_ids, lengths, expect = _batch(device)
    seq = torch.from_numpy(lengths).to(device)
    for out_dtype in (torch.int32, torch.int64):
        indptr = torch.empty(len(lengths) + 1, dtype=torch.int32, device=device)
        pt.build_indptr(seq, indptr)
        out = torch.full((int(lengths.sum()),), -9, dtype=out_dtype, device=device)
        pt.context_decode_indices(reg.rows, table, row_ids, seq, indptr, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ip = indptr.cpu().numpy()
        np.testing.assert_array_equal(ip, dec.kv_indptr(lengths))
        for b, (_, want, _) in enumerate(expect):
            np.testing.assert_array_equal(got[ip[b] : ip[b + 1]], want)


@pytest.mark.parametrize("window", [0, 1, 7, 128, 5000])
def test_window_and_dense_table_match_oracle(device, window):
    table, reg, row_ids, lengths, expect = _batch(device, seed=1)
    seq = torch.from_numpy(lengths).to(device)
    want_len = dec.window_lengths(reg.rows.cpu().numpy(), row_ids.cpu().numpy(), lengths, window, memory=reg.host)
    indptr_buf = torch.zeros(len(lengths) + 8, dtype=torch.int32, device=device)
    out = torch.zeros(int(want_len.sum()) + 5, dtype=torch.int64, device=device)
    indptr, got_len, _ = window_indices(reg.rows, table, row_ids, seq, window, indptr_buf, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got_len.cpu().numpy(), want_len)
    ip = indptr.cpu().numpy()
    np.testing.assert_array_equal(ip, dec.kv_indptr(want_len))
    for b, (_, full, _) in enumerate(expect):
        s = int(lengths[b]) - int(want_len[b])
        np.testing.assert_array_equal(out.cpu().numpy()[ip[b] : ip[b + 1]], full[s:])
    # dense page-one table form (FA3 style)
    dense = torch.full((len(lengths), 3000), -1, dtype=torch.int32, device=device)
    got = dense_indices(reg.rows, table, row_ids, seq, dense, window=window)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want_len)
    d = dense.cpu().numpy()
    for b, (_, full, _) in enumerate(expect):
        s = int(lengths[b]) - int(want_len[b])
        np.testing.assert_array_equal(d[b, : want_len[b]], full[s:])


@pytest.mark.parametrize("seed", range(8))
def test_random_registry_batches(device, seed):
    # seeded random batches of ordinary and compacted rows: full read
    # indices (int32 / int64) and a random window, list and dense forms
    rng = np.random.default_rng(800 + seed)
    batch = int(rng.integers(1, 41))
    window = int(rng.choice([0, 1, int(rng.integers(2, 3000))]))
    print(f"registry random {seed}: batch={batch} window={window}", flush=True)
    table, reg, row_ids, lengths, expect = _batch(device, seed=800 + seed, batch=batch)
    seq = torch.from_numpy(lengths).to(device)
    indptr = torch.empty(batch + 1, dtype=torch.int32, device=device)
    pt.build_indptr(seq, indptr)
    out = torch.full((int(lengths.sum()),), -9, dtype=[torch.int32, torch.int64][seed % 2], device=device)
    pt.context_decode_indices(reg.rows, table, row_ids, seq, indptr, out)
    want_len = dec.window_lengths(reg.rows.cpu().numpy(), row_ids.cpu().numpy(), lengths, window, memory=reg.host)
    wbuf = torch.zeros(batch + 8, dtype=torch.int32, device=device)
    wout = torch.zeros(int(want_len.sum()) + 5, dtype=torch.int64, device=device)
    wptr, got_len, _ = window_indices(reg.rows, table, row_ids, seq, window, wbuf, wout)
    dense = torch.full((batch, 3000), -1, dtype=torch.int32, device=device)
    dlen = dense_indices(reg.rows, table, row_ids, seq, dense, window=window)
    torch.cuda.synchronize()
    ip, got = indptr.cpu().numpy(), out.cpu().numpy()
    np.testing.assert_array_equal(ip, dec.kv_indptr(lengths))
    np.testing.assert_array_equal(got_len.cpu().numpy(), want_len)
    np.testing.assert_array_equal(dlen.cpu().numpy(), want_len)
    wip, wgot, d = wptr.cpu().numpy(), wout.cpu().numpy(), dense.cpu().numpy()
    np.testing.assert_array_equal(wip, dec.kv_indptr(want_len))
    for b, (_, full, _) in enumerate(expect):
        np.testing.assert_array_equal(got[ip[b] : ip[b + 1]], full, err_msg=f"request {b}")
        s = int(lengths[b]) - int(want_len[b])
        np.testing.assert_array_equal(wgot[wip[b] : wip[b + 1]], full[s:], err_msg=f"window of request {b}")
        np.testing.assert_array_equal(d[b, : want_len[b]], full[s:], err_msg=f"dense row {b}")


def test_mapping_translation_and_row_slots(device):
    table, reg, row_ids, lengths, expect = _batch(device, seed=2, batch=6)
    mapping = (torch.arange(10**7, dtype=torch.int64) * 5 + 3).to(device)
    seq = torch.from_numpy(lengths).to(device)
    indptr = torch.empty(len(lengths) + 1, dtype=torch.int64, device=device)
    pt.build_indptr(seq, indptr)
    out = torch.zeros(int(lengths.sum()), dtype=torch.int64, device=device)
    pt.context_decode_indices(reg.rows, table, row_ids.to(torch.int32), seq, indptr, out, mapping=mapping,
                              multiplier=2)
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
    """compact_rows outputs serve directly as registry rows (no host round trip)."""
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
    kept_off = np.concatenate(([0], np.cumsum(inputs.kept)))
    rows = []
    for b, lay in enumerate(layouts):
        raw_ptr = out.raw_indices.data_ptr() + 4 * int(kept_off[b])
        pos_ptr = out.active_positions.data_ptr() + 4 * int(kept_off[b])
        rows.append((raw_ptr, pos_ptr, w.lengths[b], inputs.kept[b], lay.next_position, 0))
    registry = torch.tensor(rows, dtype=torch.int64).to(device)
    seq = torch.tensor([k + 1 for k in inputs.kept], dtype=torch.int64, device=device)
    indptr = torch.empty(w.n_requests + 1, dtype=torch.int32, device=device)
    pt.build_indptr(seq, indptr)
    kv = torch.empty(int(seq.sum()), dtype=torch.int32, device=device)
    # the decode layout feeds the index kernel on the device, gated by the
    # compaction's status word
    pt.context_decode_indices(registry, table, row_ids, seq, indptr, kv, status=out.status)
    torch.cuda.synchronize()
    assert tables.check_status(out) == 0
    assert torch.equal(kv, out.kv_indices)
    assert torch.equal(indptr, out.kv_indptr)


@pytest.mark.parametrize("lens_dtype,loc_dtype", [(torch.int64, torch.int64), (torch.int32, torch.int32)])
def test_extend_write_matches_numpy(device, lens_dtype, loc_dtype):
    """Extend write of request rows (prefix, then new slots) into table rows
    and, for some requests, side rows reached through row pointers."""
    rng = np.random.default_rng(7)
    pool_rows, width, batch = 12, 5000, 9
    table = torch.full((pool_rows, width), -4, dtype=torch.int32, device=device)
    side = {r: torch.full((width,), -6, dtype=torch.int32, device=device) for r in (3, 8)}
    pointers = torch.tensor([side[r].data_ptr() if r in side else table[r].data_ptr() for r in range(pool_rows)],
                            dtype=torch.int64, device=device)
    req_rows = rng.permutation(pool_rows)[:batch]
    pre = rng.integers(0, 3000, size=batch)
    pre[0] = 0
    ext = rng.integers(1, 1500, size=batch)
    seq = pre + ext
    prefixes = [torch.from_numpy(rng.integers(1, 10**6, size=max(p, 1))).to(device) for p in pre]
    loc = rng.integers(1, 10**6, size=int(ext.sum()))
    args = dict(
        req_pool_indices=torch.from_numpy(req_rows.astype(np.int64)).to(device),
        prefix_tensors=torch.tensor([t.data_ptr() for t in prefixes], dtype=torch.int64, device=device),
        pre_lens=torch.from_numpy(pre).to(lens_dtype).to(device),
        seq_lens=torch.from_numpy(seq).to(lens_dtype).to(device),
        extend_lens=torch.from_numpy(ext).to(lens_dtype).to(device),
        out_cache_loc=torch.from_numpy(loc).to(loc_dtype).to(device))
    want_table = table.cpu().numpy().copy()
    want_side = {r: t.cpu().numpy().copy() for r, t in side.items()}
    start = np.concatenate(([0], np.cumsum(ext)))
    for b, r in enumerate(req_rows):
        row = want_side[r] if r in side else want_table[r]
        row[: pre[b]] = prefixes[b].cpu().numpy()[: pre[b]]
        row[pre[b] : seq[b]] = loc[start[b] : start[b + 1]]
    pt.write_req_to_token_pool(table, row_pointers=pointers, **args)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(table.cpu().numpy(), want_table)  # side-row requests leave the table alone
    for r, t in side.items():
        np.testing.assert_array_equal(t.cpu().numpy(), want_side[r])
    # without row pointers every request writes its table row
    table2 = torch.full((pool_rows, width), -4, dtype=torch.int32, device=device)
    want2 = table2.cpu().numpy().copy()
    for b, r in enumerate(req_rows):
        want2[r, : pre[b]] = prefixes[b].cpu().numpy()[: pre[b]]
        want2[r, pre[b] : seq[b]] = loc[start[b] : start[b + 1]]
    pt.write_req_to_token_pool(table2, **args)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(table2.cpu().numpy(), want2)
