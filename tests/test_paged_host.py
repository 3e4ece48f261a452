"""Host side of the paged copy-on-write path: page assignment invariants of the
shared-prefix workloads and the per-request bases packed for the kernel."""

import numpy as np
import pytest
import torch

from akv_amd import synth, tables
from oracle import paging as pg


def _layouts(w):
    return synth.compile_layouts(w)


@pytest.mark.parametrize("groups", [None, "quarters", "singles"])
def test_assign_pages_never_hands_out_a_live_page(groups):
    w = synth.workload("llama3-cow-small")
    B = w.n_requests
    split = {None: None, "quarters": [range(i, i + 4) for i in range(0, B, 4)],
             "singles": [[b] for b in range(B)]}[groups]
    a = synth.assign_pages(w, split)
    layouts = _layouts(w)
    P = w.page_size
    old_pages = [np.unique(r.astype(np.int64) // P) for r in a.birth_rows]
    all_old = np.unique(np.concatenate(old_pages))
    assert 0 not in all_old and all_old.max() < a.pool_pages
    # the shared prefix is the same physical pages in every row
    for r in a.birth_rows:
        np.testing.assert_array_equal(r[: w.shared_prefix:P] // P, a.shared_pages)
    new_tables = [None] * B
    for g in a.groups:
        live = set()
        for b in range(B):
            live.update((new_tables[b] if new_tables[b] is not None else old_pages[b]).tolist())
        fresh = np.concatenate([a.fresh_pages[b] for b in g])
        assert len(np.unique(fresh)) == len(fresh)
        assert not live & set(fresh.tolist()), "fresh page still referenced"
        assert fresh.min(initial=1) > 0 and fresh.max(initial=0) < a.pool_pages
        for b in g:
            lay = layouts[b]
            out = pg.compact_pages(a.birth_rows[b], lay.keep_mask, lay.birth_positions, lay.positions,
                                   a.fresh_pages[b], P)
            new_tables[b] = out["page_table"].astype(np.int64)
    # the page tables at the end are disjoint apart from the shared pages kept below p0
    seen = {}
    for b, t in enumerate(new_tables):
        for p in t.tolist():
            seen.setdefault(p, []).append(b)
    shared = set(a.shared_pages.tolist())
    assert all(len(v) == 1 or p in shared for p, v in seen.items())


def test_grouping_bounds_the_pool():
    w = synth.workload("llama3-cow-16")
    one = synth.assign_pages(w)
    four = synth.assign_pages(w, [range(i, i + 4) for i in range(0, 16, 4)])
    old = 1 + w.shared_prefix // w.page_size + sum(-(-(n - w.shared_prefix) // w.page_size) for n in w.lengths)
    fresh = sum(d[2] for d in synth.paged_demand(w))
    assert one.pool_pages == old + fresh
    assert old < four.pool_pages < one.pool_pages
    # 128 KiB of K+V per token over 32 layers: four groups fit 288 GB of HBM
    assert four.pool_pages * 16 * 131072 < 240e9


def test_pack_paged_inputs_bases():
    w = synth.workload("llama3-cow-small")
    layouts = _layouts(w)
    P = w.page_size
    inp = tables.pack_paged_inputs(layouts, P, "cpu")
    bases = inp.bases.numpy()
    B = w.n_requests
    assert bases.shape == (6, B + 1)
    kept = [int(l.keep_mask.sum()) for l in layouts]
    n = list(w.lengths)
    p0 = [pg.first_copied_page(l.keep_mask, P) for l in layouts]
    np.testing.assert_array_equal(bases[0, :B], np.array(p0) * P)
    np.testing.assert_array_equal(np.diff(bases[1]), kept)
    np.testing.assert_array_equal(np.diff(bases[2]), [k - q * P for k, q in zip(kept, p0)])
    np.testing.assert_array_equal(np.diff(bases[3]), [pg.fresh_page_count(k, m, l.keep_mask, P)
                                                      for k, m, l in zip(kept, n, layouts)])
    np.testing.assert_array_equal(np.diff(bases[4]), [-(-k // P) for k in kept])
    np.testing.assert_array_equal(np.diff(bases[5]), [-(-m // P) - q for m, q in zip(n, p0)])
    np.testing.assert_array_equal(inp.req_offsets.numpy(), np.concatenate(([0], np.cumsum(n))))
    flat_keep = np.concatenate([np.asarray(l.keep_mask) for l in layouts])
    np.testing.assert_array_equal(inp.keep.numpy().astype(bool), flat_keep)
    np.testing.assert_array_equal(inp.final_positions.numpy(),
                                  np.concatenate([np.asarray(l.positions) for l in layouts]))


def test_pack_paged_inputs_rejects_uncompacted_positions():
    lay = synth.compile_context_layout(
        token_ids=torch.arange(40, dtype=torch.int32),
        drop_insert_offsets=torch.tensor([40], dtype=torch.int32),
        drop_range_offsets=torch.tensor([0, 1], dtype=torch.int32),
        drop_ranges=torch.tensor([3, 9], dtype=torch.int32),
        reposition_raw_boundaries=torch.tensor([], dtype=torch.int32),
        reposition_insert_offsets=torch.tensor([], dtype=torch.int32),
    )
    with pytest.raises(ValueError, match="compact final positions"):
        tables.pack_paged_inputs([lay], 16, "cpu")


def test_pack_paged_inputs_rejects_prefix_births_off_rank():
    """Pages before the first drop stay in place, unrotated, so their tokens
    must already sit at their final positions.  Compiled event programs
    always satisfy this (no drop precedes those tokens); a hand-made layout
    that does not is rejected instead of leaving stale rotations behind."""
    from types import SimpleNamespace

    n, P = 64, 16
    keep = np.ones(n, dtype=bool)
    keep[40:44] = False
    final = np.where(keep, np.cumsum(keep) - 1, -1).astype(np.int32)
    birth = np.arange(n, dtype=np.int32)
    ok = SimpleNamespace(keep_mask=keep, positions=final, birth_positions=birth)
    tables.pack_paged_inputs([ok], P, "cpu")
    bad_birth = birth.copy()
    bad_birth[5] = 7
    bad = SimpleNamespace(keep_mask=keep, positions=final, birth_positions=bad_birth)
    with pytest.raises(ValueError, match="birth positions must equal their ranks"):
        tables.pack_paged_inputs([bad], P, "cpu")
    # the same token past the first copied page is a copy with pair (birth, rank): accepted
    late = birth.copy()
    late[50] = 52
    tables.pack_paged_inputs([SimpleNamespace(keep_mask=keep, positions=final, birth_positions=late)], P, "cpu")


@pytest.mark.parametrize("n", [37, 48])
def test_pack_paged_inputs_undropped_request(n):
    # nothing dropped: p0 lies past the last page, so p0 * P may exceed a
    # ragged length; nothing is copied, released or handed out
    P = 16
    keep = np.ones(n, dtype=bool)
    pos = np.arange(n, dtype=np.int32)
    from types import SimpleNamespace

    inp = tables.pack_paged_inputs([SimpleNamespace(keep_mask=keep, positions=pos, birth_positions=pos)], P, "cpu")
    bases = inp.bases.numpy()
    assert bases[0, 0] == -(-n // P) * P
    assert bases[2, 1] == bases[3, 1] == bases[5, 1] == 0
    assert bases[4, 1] == -(-n // P)
    assert inp.fresh_pages == (0,)
