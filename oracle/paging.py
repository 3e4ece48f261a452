"""CPU oracle of page-granular Drop + Reposition with copy-on-write.

The reference supports only page size 1 (``context_reposition.py:153-154``);
this is the paged extension's specification, restated simply:

* a request's raw row holds token slots ``page * P + offset`` (page-aligned);
* after Drop + Reposition the kept tokens sit at final positions
  ``0 .. kept - 1`` (their rank) and are packed page-dense by rank;
* ``p0 = first dropped raw token // P`` (past the last page when nothing is
  dropped): logical pages ``< p0`` keep their physical pages (shared prefix
  pages stay shared, no copy);
* every kept token of rank ``r >= p0 * P`` moves out of place to
  ``fresh_pages[r // P - p0] * P + r % P`` -- a copy-on-write for pages that
  other requests still reference, and hazard-free for private ones; the copy
  carries ``(birth position, r)``, so tokens whose position did not change
  are bit copies and the others are re-rotated;
* the request releases its old pages of logical index ``>= p0`` (raw order);
* its new page table is the old pages ``< p0`` then the fresh pages.

Pinned by (``tests/test_oracle_paging.py``): with ``P = 1`` it equals the
single-stage closed form of ``oracle.occurrence.closed_form`` (terminal
row, retired slots, copy lists); page conservation (released + kept =
old + fresh, no page in two places); every kept token's new slot sits at
page ``r // P`` offset ``r % P`` of the new page table.
"""

import numpy as np


def first_drop(keep):
    dropped = np.flatnonzero(~np.asarray(keep, dtype=bool))
    return int(dropped[0]) if len(dropped) else len(keep)


def first_copied_page(keep, page_size):
    """p0: the page of the first dropped token; no drop -> past the last page."""
    keep = np.asarray(keep, dtype=bool)
    if keep.all():
        return -(-len(keep) // page_size)
    return first_drop(keep) // page_size


def fresh_page_count(n_kept, n, keep, page_size):
    p0 = first_copied_page(keep, page_size)
    return max(0, -(-n_kept // page_size) - p0)


def compact_pages(row, keep, birth_positions, final_positions, fresh_pages, page_size):
    """Terminal row, copy lists, released pages and new page table of one request."""
    row = np.asarray(row, dtype=np.int64)
    keep = np.asarray(keep, dtype=bool)
    birth = np.asarray(birth_positions, dtype=np.int64)
    final = np.asarray(final_positions, dtype=np.int64)
    n = len(row)
    P = page_size
    kept_idx = np.flatnonzero(keep)
    if not np.array_equal(final[kept_idx], np.arange(len(kept_idx))):
        raise ValueError("paged compaction needs compact final positions (0 .. kept - 1)")
    p0 = first_copied_page(keep, P)
    # the pages before the first drop stay in place, unrotated
    if not np.array_equal(birth[: p0 * P], np.arange(min(n, p0 * P))):
        raise ValueError("pages kept in place need birth positions equal to their ranks")
    fresh_pages = np.asarray(fresh_pages, dtype=np.int64)
    need = max(0, -(-len(kept_idx) // P) - p0)
    if len(fresh_pages) != need:
        raise ValueError(f"need {need} fresh pages, got {len(fresh_pages)}")
    terminal = np.where(keep, row, -1)
    r = final[kept_idx]
    copied = r >= p0 * P
    t_c = kept_idx[copied]
    r_c = r[copied]
    dst = fresh_pages[r_c // P - p0] * P + r_c % P
    terminal[t_c] = dst
    released = row[np.arange(p0 * P, n, P)] // P if n > p0 * P else np.zeros(0, np.int64)
    n_pages = -(-len(kept_idx) // P)
    table = np.concatenate((row[np.arange(0, p0 * P, P)] // P, fresh_pages))[:n_pages]
    return {
        "terminal_row": terminal,
        "copy_source_slots": row[t_c].astype(np.int32),
        "copy_destination_slots": dst.astype(np.int32),
        "copy_position_pairs": np.stack((birth[t_c], r_c), 1).astype(np.int32),
        "released_pages": released,
        "page_table": table,
        "raw_indices": kept_idx.astype(np.int32),
        "active_positions": r.astype(np.int32),
        "active_slots": terminal[kept_idx],
        "first_copied_page": p0,
    }
