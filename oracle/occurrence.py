"""CPU restatement of the final-forward slot ownership (tables + freed list).

For a fresh request whose whole prompt is computed in one forward
(``query_start = 0``, ``query_end = n``, every slot request-owned), this
module restates, in numpy:

* ``compile_occurrence_window``
  (``akv/system/sglang/srt/context_system/occurrence.py:112-265``),
* ``plan_occurrence_materialization`` (``:341-466``),
* ``OccurrenceState.advance`` for an empty predecessor state (``:632-755``),
* ``OccurrenceState.terminal_slots`` (``:757-767``),
* ``ContextDecodeLayout.from_layout`` (``:47-66``) and the compacted active
  row of ``request_active_slots``
  (``akv/system/sglang/srt/disaggregation/context_transfer.py:110-128``).

Pinned by (``tests/test_oracle_occurrence.py``): the closed form of the
single-stage case -- terminal row ``keep ? (moved ? fresh[rank] : birth) : -1``,
retired = birth slots of dropped-or-moved tokens in raw order, copy pairs
``(birth, final)`` -- on random programs, plus the conservation invariants
multiset(retired) + multiset(row != -1) = multiset(birth) + multiset(fresh),
``len(retired) = n - kept + M`` and no duplicate live slot.
"""

from itertools import pairwise

import numpy as np


def compile_window(layout, visible_until, query_start=0, query_end=None):
    """Occurrence window of the queries ``[query_start, query_end)``.

    Occurrences ``[0, n)`` are the birth versions of every raw token; then,
    segment by segment, the versions a query reads that differ from the last
    materialised one; last the terminal versions that still differ.  Segments
    split each stage's queries wherever a token's visibility ends.
    """
    birth = layout.birth_positions.astype(np.int64)
    stages = layout.birth_stages.astype(np.int64)
    offsets = layout.transition_offsets.astype(np.int64)
    changed = layout.transition_raw_tokens.astype(np.int64)
    new = layout.transition_new_positions.astype(np.int64)
    expiry = np.asarray(visible_until, dtype=np.int64)
    n = len(birth)
    if query_end is None:
        query_end = n
    if not 0 <= query_start < query_end <= n:
        raise ValueError("Occurrence query window is outside the raw prompt.")
    stage_count = len(offsets) - 1
    raw = np.arange(n, dtype=np.int64)
    if np.any(expiry <= raw):
        raise ValueError("A token cannot become invisible before it has been computed.")
    bounds = np.searchsorted(stages, np.arange(stage_count + 2))
    current_ids = raw.copy()
    current_pos = birth.copy()
    materialized = birth.copy()
    raw_parts, pos_parts = [raw], [birth]
    next_id = n
    starts, ends, keys, key_offsets = [], [], [], [0]

    def materialize(idx):
        nonlocal next_id
        stale = idx[materialized[idx] != current_pos[idx]]
        if not len(stale):
            return
        raw_parts.append(stale)
        pos_parts.append(current_pos[stale])
        current_ids[stale] = np.arange(next_id, next_id + len(stale))
        materialized[stale] = current_pos[stale]
        next_id += len(stale)

    for stage in range(stage_count + 1):
        if stage:
            lo, hi = int(offsets[stage - 1]), int(offsets[stage])
            current_pos[changed[lo:hi]] = new[lo:hi]
        a = max(query_start, int(bounds[stage]))
        b = min(query_end, int(bounds[stage + 1]))
        if a >= b:
            continue
        inner = expiry[:b]
        cuts = [a, *np.unique(inner[(inner > a) & (inner < b)]).tolist(), b]
        for start, end in pairwise(cuts):
            alive = raw[:start][expiry[:start] > start]
            materialize(alive)
            selected = np.concatenate((current_ids[alive], raw[start:end]))
            starts.append(start)
            ends.append(end)
            keys.append(selected)
            key_offsets.append(key_offsets[-1] + len(selected))
    if not np.array_equal(current_pos, layout.positions.astype(np.int64)):
        raise ValueError(
            "Compact occurrence transitions disagree with terminal Radix positions."
        )
    materialize(raw)
    return {
        "raw": np.concatenate(raw_parts),
        "pos": np.concatenate(pos_parts),
        "birth": raw,
        "terminal": current_ids,
        "keys": np.concatenate(keys) if keys else np.zeros(0, np.int64),
        "starts": np.asarray(starts, dtype=np.int64),
        "ends": np.asarray(ends, dtype=np.int64),
        "key_offsets": np.asarray(key_offsets, dtype=np.int64),
    }


def plan_final_forward(layout, visible_until):
    """Allocation plan for the whole-prompt forward of a fresh request."""
    w = compile_window(layout, visible_until)
    raw, pos, birth, terminal = w["raw"], w["pos"], w["birth"], w["terminal"]
    n = len(birth)
    count = len(raw)
    canonical_pos = pos[birth]
    read = np.zeros(count, dtype=bool)
    read[w["keys"]] = True
    required = read.copy()
    required[birth] = True
    keep = layout.keep_mask.astype(bool)
    publish_raw = np.flatnonzero(keep)
    publish_ids = terminal[publish_raw]
    required[publish_ids] = True
    ids = np.flatnonzero(required)
    reuse = canonical_pos[raw[ids]] == pos[ids]
    rows = np.full(count, -1, dtype=np.int64)
    rows[ids[reuse]] = raw[ids[reuse]]
    allocated = ids[~reuse]
    copied_raw = raw[allocated]
    pairs = np.column_stack((canonical_pos[copied_raw], pos[allocated])).astype(np.int32)
    retained = np.full(n, -1, dtype=np.int64)
    retained[publish_raw] = publish_ids
    return {
        "window": w,
        "source_rows": rows,
        "allocated": allocated,
        "copy_rows": copied_raw,
        "pairs": pairs,
        "terminal_occurrences": retained,
        "extra_page_count": len(allocated),
    }


def advance_final_forward(layout, plan, query_slots, extra_slots):
    """Bind birth + fresh slots; returns copy lists, retired slots, terminal row."""
    query_slots = np.asarray(query_slots, dtype=np.int64)
    extra_slots = np.asarray(extra_slots, dtype=np.int64)
    n = len(query_slots)
    if len(extra_slots) != plan["extra_page_count"]:
        raise ValueError("Context admission does not cover the selected window")
    all_slots = np.concatenate((query_slots, extra_slots))
    rows = plan["source_rows"]
    occurrences = np.full(len(rows), -1, dtype=np.int64)
    reuse = rows >= 0
    occurrences[reuse] = rows[reuse]  # canonical row r is all_slots index r
    occurrences[plan["allocated"]] = np.arange(n, len(all_slots))
    selected = plan["terminal_occurrences"]
    kept = selected >= 0
    terminal = np.full(n, -1, dtype=np.int64)
    terminal[kept] = occurrences[selected[kept]]
    live = np.zeros(len(all_slots), dtype=bool)
    live[terminal[kept]] = True
    retired = np.flatnonzero(~live)
    row = np.full(n, -1, dtype=np.int64)
    row[kept] = all_slots[terminal[kept]]
    return {
        "copy_source_slots": all_slots[plan["copy_rows"]].astype(np.int32),
        "copy_destination_slots": all_slots[occurrences[plan["allocated"]]].astype(np.int32),
        "copy_position_pairs": plan["pairs"],
        "retired_slots": all_slots[retired],
        "terminal_row": row,
        "occurrence_slots": all_slots[np.maximum(occurrences, 0)],
    }


def decode_layout(layout):
    """``ContextDecodeLayout.from_layout``: kept raw ids and their positions."""
    raw = np.flatnonzero(layout.keep_mask).astype(np.int32)
    positions = layout.positions[raw].astype(np.int32)
    if np.any(np.diff(positions.astype(np.int64)) <= 0):
        raise ValueError("Active decode positions must be strictly increasing")
    return raw, positions


def closed_form(birth_row, keep, birth_positions, final_positions, fresh):
    """Terminal row / retired / copies of a single-owner final forward.

    A kept token whose final position differs from its birth position is
    "moved": it takes the next fresh slot (raw order) and is copied from its
    birth slot with pair (birth, final).  Retired = birth slots of dropped or
    moved tokens, in raw order.
    """
    birth_row = np.asarray(birth_row, dtype=np.int64)
    keep = np.asarray(keep, dtype=bool)
    moved = keep & (np.asarray(birth_positions) != np.asarray(final_positions))
    fresh = np.asarray(fresh, dtype=np.int64)
    if int(moved.sum()) != len(fresh):
        raise ValueError("fresh slot count does not match the moved tokens")
    row = np.where(keep, birth_row, -1)
    row[moved] = fresh
    retired = birth_row[~keep | moved]
    pairs = np.column_stack(
        (np.asarray(birth_positions)[moved], np.asarray(final_positions)[moved])
    ).astype(np.int32)
    raw_indices = np.flatnonzero(keep).astype(np.int32)
    return {
        "terminal_row": row,
        "retired_slots": retired,
        "copy_source_slots": birth_row[moved].astype(np.int32),
        "copy_destination_slots": fresh.astype(np.int32),
        "copy_position_pairs": pairs,
        "raw_indices": raw_indices,
        "active_positions": np.asarray(final_positions)[raw_indices].astype(np.int32),
        "active_slots": row[raw_indices],
    }
