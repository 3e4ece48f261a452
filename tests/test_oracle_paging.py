"""Pins oracle.paging: page size 1 equals the single-stage closed form;
page conservation and rank-aligned placement for page size 16."""

import numpy as np

from oracle import events as ev
from oracle import occurrence as occ
from oracle import paging as pg


def _request(rng, n, page_size, pages):
    k = int(rng.integers(1, 4))
    cuts = np.sort(rng.choice(np.arange(n + 1), size=2 * k, replace=False))
    spans = [(int(cuts[2 * j]), int(cuts[2 * j + 1])) for j in range(k)]
    lay = ev.compile_context_layout(np.arange(n), np.array([n]), np.array([0, k]),
                                    np.array([x for s in spans for x in s]), np.array([n - 1]), np.array([n]))
    if not lay.keep_mask.any():
        return None
    n_pages = -(-n // page_size)
    phys = pages[:n_pages]
    row = (phys[np.arange(n) // page_size] * page_size + np.arange(n) % page_size).astype(np.int64)
    return lay, row


def test_page_one_equals_single_stage_closed_form():
    rng = np.random.default_rng(0)
    for _ in range(50):
        n = int(rng.integers(4, 300))
        pages = rng.permutation(np.arange(1, 4 * n))
        got = _request(rng, n, 1, pages)
        if got is None:
            continue
        lay, row = got
        kept = int(lay.keep_mask.sum())
        fresh_n = pg.fresh_page_count(kept, n, lay.keep_mask, 1)
        fresh = pages[n : n + fresh_n]
        paged = pg.compact_pages(row, lay.keep_mask, lay.birth_positions, lay.positions, fresh, 1)
        moved = lay.keep_mask & (lay.birth_positions != lay.positions)
        assert fresh_n >= int(moved.sum())
        # with P = 1 the pages from the first drop on are exactly the moved
        # tokens' slots plus the dropped ones; the copies of unmoved tokens
        # after p0 do not exist (every kept token after the first drop moves)
        assert fresh_n == int(moved.sum())
        cf = occ.closed_form(row, lay.keep_mask, lay.birth_positions, lay.positions, fresh)
        np.testing.assert_array_equal(paged["terminal_row"], cf["terminal_row"])
        np.testing.assert_array_equal(paged["released_pages"], cf["retired_slots"])
        np.testing.assert_array_equal(paged["copy_source_slots"], cf["copy_source_slots"])
        np.testing.assert_array_equal(paged["copy_destination_slots"], cf["copy_destination_slots"])
        np.testing.assert_array_equal(paged["copy_position_pairs"], cf["copy_position_pairs"])


def test_page_sixteen_conservation_and_placement():
    rng = np.random.default_rng(1)
    P = 16
    for _ in range(40):
        n = int(rng.integers(20, 2000))
        pages = rng.permutation(np.arange(1, 4 * n))
        got = _request(rng, n, P, pages)
        if got is None:
            continue
        lay, row = got
        kept = int(lay.keep_mask.sum())
        n_pages = -(-n // P)
        fresh_n = pg.fresh_page_count(kept, n, lay.keep_mask, P)
        fresh = pages[n_pages : n_pages + fresh_n]
        out = pg.compact_pages(row, lay.keep_mask, lay.birth_positions, lay.positions, fresh, P)
        p0 = out["first_copied_page"]
        old = row[np.arange(0, n, P)] // P
        kept_pages = out["page_table"]
        # released + still-used old pages = all old pages; fresh pages all used
        still = set(kept_pages[:p0].tolist())
        assert still | set(out["released_pages"].tolist()) == set(old.tolist())
        assert not (still & set(out["released_pages"].tolist()))
        assert set(kept_pages[p0:].tolist()) == set(fresh.tolist())
        # kept token of rank r sits at page table[r // P], offset r % P
        slots = out["active_slots"]
        r = np.arange(kept)
        np.testing.assert_array_equal(slots // P, kept_pages[r // P])
        np.testing.assert_array_equal(slots % P, r % P)
        # copies: exactly the kept tokens of rank >= p0 * P, unchanged
        # positions only for ranks below the first dropped token
        pairs = out["copy_position_pairs"]
        assert len(pairs) == max(0, kept - p0 * P)
        first = pg.first_drop(lay.keep_mask)
        same = pairs[:, 0] == pairs[:, 1]
        np.testing.assert_array_equal(same, pairs[:, 1] < first)


def test_pages_kept_in_place_need_birth_at_rank():
    import pytest

    n, P = 64, 16
    keep = np.ones(n, dtype=bool)
    keep[40:44] = False
    final = np.where(keep, np.cumsum(keep) - 1, -1)
    row = np.arange(1, n + 1) * 1
    birth = np.arange(n)
    fresh = np.array([100])  # kept 60 -> 4 pages, p0 = 2 -> 2 fresh pages
    with pytest.raises(ValueError, match="need 2 fresh pages"):
        pg.compact_pages(row, keep, birth, final, fresh, P)
    out = pg.compact_pages(row, keep, birth, final, np.array([100, 101]), P)
    assert out["first_copied_page"] == 2
    bad = birth.copy()
    bad[3] = 9
    with pytest.raises(ValueError, match="birth positions equal to their ranks"):
        pg.compact_pages(row, keep, bad, final, np.array([100, 101]), P)
