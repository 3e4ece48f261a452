"""GPU parity of the batched page-table compaction against the oracle.

Integer outputs must be bit-exact: terminal rows (in place), retired slots,
copy lists, decode layouts, compacted rows / kv_indices and kv_indptr.
"""

import ctypes

import numpy as np
import pytest
import torch

from akv_amd import _lib, synth, tables
from oracle import occurrence as occ

pytestmark = pytest.mark.gpu


def _setup(device, w, layouts, *, generated=None, side_rows=False, width_extra=8):
    slots = synth.assign_slots(w, layouts)
    inputs = tables.pack_compaction_inputs(layouts, device)
    width = max(w.lengths) + width_extra
    pool_rows = w.n_requests + 3
    table = torch.full((pool_rows, width), -5, dtype=torch.int32)
    rng = np.random.default_rng(w.seed)
    req_rows = rng.permutation(np.arange(pool_rows))[: w.n_requests]
    gen = generated if generated is not None else [0] * w.n_requests
    tails = []
    for b, row in enumerate(req_rows):
        n = w.lengths[b]
        table[row, :n] = torch.from_numpy(slots.birth_rows[b])
        tail = rng.integers(1, 10**6, size=gen[b]).astype(np.int32)
        table[row, n : n + gen[b]] = torch.from_numpy(tail)
        tails.append(tail)
    table = table.to(device)
    row_pointers = None
    side = {}
    if side_rows:
        # every request lives in its own side row, outside the table
        ptrs = torch.tensor([table[r].data_ptr() for r in range(pool_rows)], dtype=torch.int64)
        for b, row in enumerate(req_rows):
            side[row] = table[row].clone()
            ptrs[row] = side[row].data_ptr()
        row_pointers = ptrs.to(device)
    fresh = torch.from_numpy(np.concatenate(slots.fresh).astype(np.int32) if slots.fresh else np.zeros(0, np.int32)).to(device)
    return slots, inputs, table, torch.from_numpy(req_rows.astype(np.int64)).to(device), fresh, row_pointers, side, tails


def _check(w, layouts, slots, out, rows_after, tails, gen):
    kept_off = moved_off = retired_off = kv_off = 0
    indptr = out.kv_indptr.cpu().numpy() if out.kv_indptr is not None else None
    counts = out.counts.cpu().numpy()
    last_page = out.last_page_len.cpu().numpy() if out.last_page_len is not None else None
    for b, lay in enumerate(layouts):
        want = occ.closed_form(slots.birth_rows[b], lay.keep_mask.numpy(), lay.birth_positions.numpy(),
                               lay.positions.numpy(), slots.fresh[b])
        n = w.lengths[b]
        kept = len(want["raw_indices"])
        moved = len(want["copy_source_slots"])
        retired = len(want["retired_slots"])
        np.testing.assert_array_equal(rows_after[b][:n], want["terminal_row"], err_msg=f"row {b}")
        np.testing.assert_array_equal(out.retired.cpu().numpy()[retired_off : retired_off + retired], want["retired_slots"])
        np.testing.assert_array_equal(out.copy_src.cpu().numpy()[moved_off : moved_off + moved], want["copy_source_slots"])
        np.testing.assert_array_equal(out.copy_dst.cpu().numpy()[moved_off : moved_off + moved], want["copy_destination_slots"])
        np.testing.assert_array_equal(out.copy_pairs.cpu().numpy()[moved_off : moved_off + moved], want["copy_position_pairs"])
        np.testing.assert_array_equal(out.raw_indices.cpu().numpy()[kept_off : kept_off + kept], want["raw_indices"])
        np.testing.assert_array_equal(out.active_positions.cpu().numpy()[kept_off : kept_off + kept], want["active_positions"])
        assert counts[b].tolist() == [kept, moved, retired]
        if last_page is not None:
            assert last_page[b] == (1 if kept + gen[b] > 0 else 0)
        if out.kv_indices is not None:
            assert indptr[b] == kv_off
            seg = out.kv_indices.cpu().numpy()[kv_off : kv_off + kept + gen[b]]
            np.testing.assert_array_equal(seg, np.concatenate((want["active_slots"], tails[b])))
            kv_off += kept + gen[b]
        kept_off += kept
        moved_off += moved
        retired_off += retired
    if indptr is not None:
        assert indptr[-1] == kv_off
    assert out.status.item() == 0


def _run(device, w, *, generated=None, side_rows=False):
    layouts = synth.compile_layouts(w)
    slots, inputs, table, req_rows, fresh, row_pointers, side, tails = _setup(
        device, w, layouts, generated=generated, side_rows=side_rows)
    gen = generated if generated is not None else [0] * w.n_requests
    out = tables.allocate_outputs(inputs, device, generated_total=sum(gen))
    gen_t = torch.tensor(gen, dtype=torch.int32, device=device) if generated is not None else None
    table_before = table.clone()
    tables.compact_rows(inputs, table, req_rows, fresh, out, row_pointers=row_pointers, generated=gen_t)
    torch.cuda.synchronize()
    rows = req_rows.cpu().numpy()
    if side_rows:
        rows_after = [side[r].cpu().numpy() for r in rows]
        # with side rows the table itself is untouched
        assert torch.equal(table, table_before)
    else:
        rows_after = [table[r].cpu().numpy() for r in rows]
    _check(w, layouts, slots, out, rows_after, tails, gen)
    return out


def test_tiny_single_request(device):
    _run(device, synth.workload("tiny"))


def test_gpt_oss_32k(device):
    _run(device, synth.workload("gpt-oss-32k"), generated=[1])


def test_ragged_batch_64(device):
    w = synth.workload("ragged-64")
    _run(device, w, generated=[int(x) for x in np.random.default_rng(5).integers(1, 9, size=w.n_requests)])


def test_side_rows_and_edge_requests(device):
    model = synth.TINY
    # no drop; drop only at the tail (ignored Reposition); drop at the head;
    # almost everything dropped; a 1-token request; a tile-boundary length
    lengths = (50, 64, 70, 5000, 1, 4096 + 17)
    spans = ((), ((60, 64),), ((0, 10),), ((1, 4999),), (), ((4095, 4097), (4100, 4101)))
    w = synth.Workload("edges", model, lengths, spans, seed=11, table_positions=5000, pool_slots=40000)
    _run(device, w, side_rows=True, generated=[2, 0, 1, 3, 1, 0])


def test_many_small_requests(device):
    # 5000 requests of 1-40 tokens: many requests start and end in every tile
    rng = np.random.default_rng(21)
    lengths, spans = [], []
    for _ in range(5000):
        n = int(rng.integers(1, 40))
        s = []
        if n > 3 and rng.random() < 0.8:
            a_, b_ = sorted(rng.choice(np.arange(n + 1), size=2, replace=False).tolist())
            if b_ - a_ < n:  # a Reposition needs at least one kept token
                s = [(a_, b_)]
        lengths.append(n)
        spans.append(tuple(s))
    w = synth.Workload("many-small", synth.TINY, tuple(lengths), tuple(spans), seed=21,
                       table_positions=64, pool_slots=4 * sum(lengths) + 1)
    _run(device, w, generated=[int(x) for x in rng.integers(0, 3, size=len(lengths))])


def test_birth_slot_vector_is_idempotent(device):
    w = synth.workload("ragged-64")
    layouts = synth.compile_layouts(w)
    slots, inputs, table, req_rows, fresh, row_pointers, side, tails = _setup(device, w, layouts)
    birth = torch.from_numpy(np.concatenate(slots.birth_rows)).to(device)
    # rows start out as garbage: with a birth vector they are only written
    table.fill_(-77)
    out = tables.allocate_outputs(inputs, device, generated_total=0)
    gen0 = torch.zeros(w.n_requests, dtype=torch.int32, device=device)
    for _ in range(2):
        tables.compact_rows(inputs, table, req_rows, fresh, out, generated=gen0, birth_slots=birth)
    torch.cuda.synchronize()
    rows_after = [table[r].cpu().numpy() for r in req_rows.cpu().numpy()]
    _check(w, layouts, slots, out, rows_after, [np.zeros(0, np.int32)] * w.n_requests, [0] * w.n_requests)


def test_fresh_count_mismatch_sets_status(device):
    w = synth.workload("tiny")
    layouts = synth.compile_layouts(w)
    slots, inputs, table, req_rows, fresh, row_pointers, side, tails = _setup(device, w, layouts)
    out = tables.allocate_outputs(inputs, device)
    # claim one fresh slot fewer than there are moved tokens
    inputs.moved = (inputs.moved[0] - 1,)
    out.copy_src, out.copy_dst = out.copy_src[:-1], out.copy_dst[:-1]
    out.copy_pairs = out.copy_pairs[:-1]
    tables.compact_rows(inputs, table, req_rows, fresh[:-1], out)
    torch.cuda.synchronize()
    assert out.status.item() == 1


def test_requests_denser_than_the_tile_window(device):
    # one-token requests: past the first tile more than 256 requests touch
    # each 256-token tile, so tokens find their request in global memory
    n = 1500
    w = synth.Workload("one-token", synth.TINY, (1,) * n, ((),) * n, seed=31, table_positions=8,
                       pool_slots=4 * n + 1)
    _run(device, w, generated=[int(x) for x in np.random.default_rng(31).integers(0, 3, size=n)])


def _path(lib, n_requests, total, largest=None):
    tile = ctypes.c_int64(0)
    launches = lib.akv_compact_launches(n_requests, total, total + n_requests if largest is None else largest,
                                        ctypes.byref(tile))
    return launches, tile.value


def test_launch_paths(device):
    """Which path each batch shape takes on this device: one launch while every
    tile fits at once and the batch stages in LDS, two launches otherwise."""
    lib = _lib.load()
    assert _path(lib, 64, 2_118_412)[0] == 1  # the ragged batch
    assert _path(lib, 1, 32_768) == (1, 256)
    assert _path(lib, 32, 32 * 32_768)[0] == 1
    assert _path(lib, 80, 80 * 65_536) == (2, 1024)  # more tiles than fit at once
    assert _path(lib, 5000, 200_000) == (2, 256)  # more requests than LDS staging
    assert _path(lib, 4, 1000, 1 << 29)[0] == 2  # a list past 32-bit byte offsets
    assert _path(lib, 0, 0) == (0, 0)


def _batch_for(lib, n_requests, want, seed):
    """A batch of n_requests whose path is `want` = (launches, tile tokens):
    the middle of the range of totals that map to it (searched on the host)."""
    hits = [t for t in range(8192, 3_200_000, 8192) if _path(lib, n_requests, t) == want]
    if not hits:
        pytest.skip(f"no batch of {n_requests} requests takes path {want} on this device")
    total = hits[len(hits) // 2]
    rng = np.random.default_rng(seed)
    cuts = np.sort(rng.choice(np.arange(1, total), size=n_requests - 1, replace=False))
    lengths = np.diff(np.concatenate(([0], cuts, [total])))
    spans = []
    for n in lengths:
        n = int(n)
        k = int(rng.integers(0, 3)) if n > 8 else 0
        starts = np.sort(rng.choice(np.arange(n - 1), size=k, replace=False)) if k else []
        req, prev = [], 0
        for a in starts:
            a = max(int(a), prev + 1 if req else 0)  # ordered, disjoint, not touching
            b = min(n, a + 1 + int(rng.integers(0, max(1, n // 8))))
            if a < b:
                req.append((a, b))
                prev = b
        spans.append(tuple(req))
    return synth.Workload(f"path-{want[0]}x{want[1]}", synth.TINY, tuple(int(n) for n in lengths), tuple(spans),
                          seed=seed, table_positions=int(lengths.max()) + 8, pool_slots=3 * total + 1)


# every tile size of the one-launch path, and of the two-launch path
@pytest.mark.parametrize("n_requests,want", [(48, (1, 256 * st)) for st in (1, 2, 3, 4, 5, 6, 8)]
                         + [(600, (2, 256)), (600, (2, 512)), (600, (2, 1024))])
def test_every_tile_size(device, n_requests, want):
    lib = _lib.load()
    w = _batch_for(lib, n_requests, want, seed=want[1] + n_requests)
    print(f"tile size {want} with {n_requests} requests, {sum(w.lengths)} tokens", flush=True)
    assert _path(lib, w.n_requests, sum(w.lengths)) == want
    _run(device, w, generated=[1] * w.n_requests)


@pytest.mark.parametrize("seed", range(12))
def test_random_batches(device, seed):
    """Seeded random batches: 1-512 requests (one- and two-launch paths,
    every tile size the total picks), up to ~1.5 M tokens, 0-3 drop spans
    and 0-3 generated tokens per request, side rows or the table; every
    output bit-exact against the oracle."""
    rng = np.random.default_rng(5000 + seed)
    n_requests = int(rng.choice([1, 2, 7, 64, 300, 512]))
    total = int(rng.integers(max(n_requests, 1000), 1_500_000))
    cuts = np.sort(rng.choice(np.arange(1, total), size=n_requests - 1, replace=False))
    lengths = np.diff(np.concatenate(([0], cuts, [total])))
    spans = []
    for n in lengths:
        n = int(n)
        k = int(rng.integers(0, 4)) if n > 8 else 0
        starts = np.sort(rng.choice(np.arange(n - 1), size=k, replace=False)) if k else []
        req, prev = [], 0
        for a in starts:
            a = max(int(a), prev + 1 if req else 0)  # ordered, disjoint, not touching
            b = min(n, a + 1 + int(rng.integers(0, max(1, n // 4))))
            if a < b:
                req.append((a, b))
                prev = b
        spans.append(tuple(req))
    w = synth.Workload(f"random-{seed}", synth.TINY, tuple(int(n) for n in lengths), tuple(spans), seed=seed,
                       table_positions=int(lengths.max()) + 8, pool_slots=3 * total + 1)
    generated = [int(g) for g in rng.integers(0, 4, n_requests)]
    side_rows = bool(rng.random() < 0.3)
    lib = _lib.load()
    print(f"random batch seed={seed}: {n_requests} requests, {total} tokens, path {_path(lib, n_requests, total)}, "
          f"side rows {side_rows}", flush=True)
    _run(device, w, generated=generated, side_rows=side_rows)


def test_prefix_over_many_tiles(device):
    # 80 x 64k tokens (two-launch path): 5000+ tiles of 1024 tokens, each
    # summing the aggregates of up to 5000 earlier tiles
    rng = np.random.default_rng(41)
    lengths = tuple([65536] * 80)
    spans = tuple(((int(a), int(a) + int(rng.integers(1, 5000))),) for a in rng.integers(0, 60000, size=80))
    w = synth.Workload("many-groups", synth.TINY, lengths, spans, seed=41, table_positions=65536,
                       pool_slots=3 * sum(lengths) + 1)
    _run(device, w, generated=[1] * 80)


def test_workspace_reused_across_batches(device):
    """One workspace serves calls of different sizes in a row, including one
    that ends with status 1."""
    big = synth.workload("ragged-64")
    small = synth.Workload("edges", synth.TINY, (50, 4096 + 17, 5), ((), ((100, 900),), ()), seed=12,
                           table_positions=5000, pool_slots=40000)
    runs = []
    for w in (big, small, big):
        layouts = synth.compile_layouts(w)
        runs.append((w, layouts, *_setup(device, w, layouts)))
    shared = tables.allocate_outputs(runs[0][3], device).workspace
    for i, (w, layouts, slots, inputs, table, req_rows, fresh, row_pointers, side, tails) in enumerate(runs):
        out = tables.allocate_outputs(inputs, device)
        out.workspace = shared
        if i == 1:
            # a mismatched call first: it sets status 1
            bad = tables.allocate_outputs(inputs, device)
            bad.workspace = shared
            inputs_bad = tables.CompactionInputs(**{**inputs.__dict__, "moved": (inputs.moved[0] + 1,) + inputs.moved[1:]})
            fresh_bad = torch.cat((fresh, fresh[:1]))
            bad.copy_src = torch.empty(len(fresh_bad), dtype=torch.int32, device=device)
            bad.copy_dst = torch.empty_like(bad.copy_src)
            bad.copy_pairs = torch.empty((len(fresh_bad), 2), dtype=torch.int32, device=device)
            tables.compact_rows(inputs_bad, table.clone(), req_rows, fresh_bad, bad)
            torch.cuda.synchronize()
            assert bad.status.item() == 1
        tables.compact_rows(inputs, table, req_rows, fresh, out)
        torch.cuda.synchronize()
        rows_after = [table[r].cpu().numpy() for r in req_rows.cpu().numpy()]
        _check(w, layouts, slots, out, rows_after, tails, [0] * w.n_requests)
