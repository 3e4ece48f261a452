"""CPU restatement of the Drop/Reposition event compiler.

Restates the two native passes of
``akv/system/sglang/kernels/ops/attention/context_plan.py`` --
``count_radix_reposition_transitions`` (``:80-208``) and
``compile_radix_reposition_layout`` (``:210-532``) -- and the Python driver
``compile_context_layout`` (``akv/system/sglang/srt/context_system/ir.py:113-274``)
as one pure-Python replay over a doubly linked list of active raw tokens.
Pure-Python loops: meant for prompts of up to a few ten-thousand tokens.

Event semantics replayed (insertion points are "before raw token i"):

* a Drop at insertion ``i`` unlinks every still-kept token of its ordered,
  disjoint, already-computed half-open ranges (``:362-403``);
* a Reposition at insertion ``i`` (raw boundary ``i - 1``) renumbers the active
  suffix that starts at the first non-compact token, continuing from the
  position of its predecessor, and records ``(raw, old, new)`` transitions
  (``:405-440``); with no non-compact token it is "ignored";
* a token is then born at ``next_position++`` (``:442-463``);
* Drop runs before Reposition at a shared insertion point (``ir.py:123-125``).

Pinned by (``tests/test_oracle_events.py``): the closed form for a single
Drop + Reposition at insertion ``n`` (``new = exclusive prefix count of keep``,
transitions = kept tokens after the first dropped token), an independent
brute-force model that recomputes every position from scratch after each event
on random multi-stage programs of up to 64 tokens, the reference's own
runtime invariants (``position > rank`` before a renumber, ``:187-188`` and
``:422-423``; count and fill passes agree, ``:529-530``; replayed transitions
reproduce terminal positions, ``occurrence.py:246-249``), and the README's
block-position example (``README.md:269-280``).
"""

from dataclasses import dataclass

import numpy as np

TOKEN_KIND = 0
DELTA_KIND = 1
REPOSITION_KIND = 2

INT32_MAX = 2**31 - 1


@dataclass
class Layout:
    positions: np.ndarray
    keep_mask: np.ndarray
    materialized_stage: np.ndarray
    birth_positions: np.ndarray
    birth_stages: np.ndarray
    transition_offsets: np.ndarray
    transition_raw_tokens: np.ndarray
    transition_old_positions: np.ndarray
    transition_new_positions: np.ndarray
    effective_reposition_stages: np.ndarray
    effective_repositions: np.ndarray
    ignored_repositions: np.ndarray
    drop_event_to_key: np.ndarray
    records: np.ndarray
    virtual_mask: np.ndarray
    key_to_token: np.ndarray
    token_to_key: np.ndarray
    next_position: int


def _as_vec(name, value):
    a = np.asarray(value)
    if a.ndim != 1 or not (a.dtype.kind in "iu" or a.size == 0):
        raise ValueError(f"{name} must be a one-dimensional CPU integer tensor.")
    a = a.astype(np.int64)
    if a.size and (a.min() < -(2**31) or a.max() >= 2**31):
        raise ValueError(f"{name} exceeds the signed int32 range.")
    return a


def _validate_events(n, drops, drop_offsets, ranges, boundaries, offsets):
    """Input checks in the order the reference's count pass makes them."""
    if not (0 <= n <= INT32_MAX):
        raise ValueError("token_count exceeds the int32 Reposition limit")
    if (
        len(drop_offsets) != len(drops) + 1
        or len(ranges) % 2
        or len(offsets) != len(boundaries)
    ):
        raise ValueError("Reposition transition-count tensor lengths are inconsistent")
    if drop_offsets[0] != 0 or drop_offsets[len(drops)] != len(ranges) // 2:
        raise ValueError("drop_range_offsets does not cover drop_ranges")
    for i in range(len(drops)):
        if not (
            0 <= drops[i] <= n
            and (i == 0 or drops[i - 1] < drops[i])
            and drop_offsets[i] < drop_offsets[i + 1]
        ):
            raise ValueError("Invalid Drop event metadata")
    for i in range(len(boundaries)):
        if not (
            offsets[i] == boundaries[i] + 1
            and 0 < offsets[i] <= n
            and (i == 0 or boundaries[i - 1] < boundaries[i])
        ):
            raise ValueError("Invalid Reposition event metadata")


def compile_context_layout(
    token_ids,
    drop_insert_offsets,
    drop_range_offsets,
    drop_ranges,
    reposition_raw_boundaries,
    reposition_insert_offsets,
):
    """Replay the event program; returns a :class:`Layout` or raises ValueError."""
    tokens = _as_vec("token_ids", token_ids)
    drops = _as_vec("drop_insert_offsets", drop_insert_offsets)
    drop_offsets = _as_vec("drop_range_offsets", drop_range_offsets)
    ranges = _as_vec("drop_ranges", drop_ranges)
    boundaries = _as_vec("reposition_raw_boundaries", reposition_raw_boundaries)
    offsets = _as_vec("reposition_insert_offsets", reposition_insert_offsets)
    n = len(tokens)
    _validate_events(n, drops, drop_offsets, ranges, boundaries, offsets)

    prev = [-1] * n
    nxt = [-1] * n
    pos = [-1] * n
    kept = [False] * n
    ready = [0] * n
    birth_pos = [0] * n
    birth_stage = [0] * n
    tail = -1
    unsettled = -1  # first active token whose position differs from its rank
    active = 0
    next_position = 0
    stage = 0
    t_raw, t_old, t_new = [], [], []
    t_offsets = [0]
    eff_stage = [-1] * len(boundaries)
    effective = [False] * len(boundaries)
    ignored = [False] * len(boundaries)
    d = r = 0
    for insertion in range(n + 1):
        if d < len(drops) and drops[d] == insertion:
            last_end = -1
            for q in range(drop_offsets[d], drop_offsets[d + 1]):
                start, end = int(ranges[2 * q]), int(ranges[2 * q + 1])
                if not (
                    0 <= start < end <= insertion
                    and (q == drop_offsets[d] or last_end < start)
                ):
                    raise ValueError(
                        "Drop ranges must be ordered, disjoint, and already materialized"
                    )
                last_end = end
                for t in range(start, end):
                    if not kept[t]:
                        continue
                    before, after = prev[t], nxt[t]
                    if before >= 0:
                        nxt[before] = after
                    if after < 0:
                        tail = before
                    else:
                        prev[after] = before
                    kept[t] = False
                    active -= 1
                    if unsettled == t:
                        unsettled = after
                    if after >= 0 and (unsettled < 0 or after < unsettled):
                        unsettled = after
            if active == 0:
                unsettled = -1
            d += 1
        if r < len(boundaries) and offsets[r] == insertion:
            if active == 0:
                raise ValueError(
                    f"Reposition at raw boundary {int(boundaries[r])} has no active tokens."
                )
            if unsettled < 0:
                ignored[r] = True
            else:
                stage += 1
                effective[r] = True
                eff_stage[r] = stage
                rank = 0 if prev[unsettled] < 0 else pos[prev[unsettled]] + 1
                t = unsettled
                while t >= 0:
                    if not pos[t] > rank:
                        raise ValueError("Non-compact active suffix invariant was violated")
                    t_raw.append(t)
                    t_old.append(pos[t])
                    t_new.append(rank)
                    pos[t] = rank
                    ready[t] = stage
                    rank += 1
                    t = nxt[t]
                next_position = active
                unsettled = -1
                t_offsets.append(len(t_raw))
            r += 1
        if insertion == n:
            continue
        t = insertion
        rank = active
        kept[t] = True
        pos[t] = next_position
        next_position += 1
        birth_pos[t] = pos[t]
        birth_stage[t] = stage
        ready[t] = stage
        prev[t] = tail
        if tail >= 0:
            nxt[tail] = t
        tail = t
        active += 1
        if unsettled < 0 and pos[t] != rank:
            unsettled = t

    # Radix key records (second pass of context_plan.py:475-522).
    records, virtual, key_token = [], [], []
    token_key = [0] * n
    drop_key = [-1] * len(drops)
    d = r = 0
    for insertion in range(n + 1):
        if d < len(drops) and drops[d] == insertion:
            drop_key[d] = len(records)
            for q in range(drop_offsets[d], drop_offsets[d + 1]):
                start, end = int(ranges[2 * q]), int(ranges[2 * q + 1])
                records.append((DELTA_KIND, -start - 1, -end - 1))
                virtual.append(True)
                key_token.append(-1)
            d += 1
        if r < len(boundaries) and offsets[r] == insertion:
            if effective[r]:
                records.append((REPOSITION_KIND, int(boundaries[r]), -1))
                virtual.append(True)
                key_token.append(-1)
            r += 1
        if insertion == n:
            continue
        token_key[insertion] = len(records)
        tid = int(tokens[insertion])
        if tid < 0 or tid > INT32_MAX:
            raise ValueError(
                f"Reposition Radix token ID {tid} is outside the non-negative int32 range."
            )
        records.append((TOKEN_KIND, tid, pos[insertion]))
        virtual.append(False)
        key_token.append(insertion)

    i32 = np.int32
    return Layout(
        positions=np.asarray(pos, dtype=i32),
        keep_mask=np.asarray(kept, dtype=bool),
        materialized_stage=np.asarray(ready, dtype=i32),
        birth_positions=np.asarray(birth_pos, dtype=i32),
        birth_stages=np.asarray(birth_stage, dtype=i32),
        transition_offsets=np.asarray(t_offsets, dtype=i32),
        transition_raw_tokens=np.asarray(t_raw, dtype=i32),
        transition_old_positions=np.asarray(t_old, dtype=i32),
        transition_new_positions=np.asarray(t_new, dtype=i32),
        effective_reposition_stages=np.asarray(eff_stage, dtype=i32),
        effective_repositions=np.asarray(effective, dtype=bool),
        ignored_repositions=np.asarray(ignored, dtype=bool),
        drop_event_to_key=np.asarray(drop_key, dtype=np.int64),
        records=np.asarray(records, dtype=i32).reshape(-1, 3),
        virtual_mask=np.asarray(virtual, dtype=bool),
        key_to_token=np.asarray(key_token, dtype=np.int64),
        token_to_key=np.asarray(token_key, dtype=np.int64),
        next_position=int(next_position),
    )


def single_stage_closed_form(n, drop_ranges):
    """Closed form of one Drop (ranges) + one Reposition, both at insertion ``n``.

    Returns ``(keep, positions, moved_raw, old, new, next_position)``.  New
    positions are the exclusive prefix count of the keep mask; the moved
    tokens are the kept tokens after the first dropped token; with no kept
    token after a dropped one the Reposition is ignored and ``next_position``
    stays ``n``.
    """
    keep = np.ones(n, dtype=bool)
    for start, end in drop_ranges:
        keep[start:end] = False
    rank = np.cumsum(keep) - keep  # exclusive prefix count
    raw = np.arange(n)
    dropped = np.flatnonzero(~keep)
    if len(dropped):
        moved = raw[keep & (raw > dropped[0])]
    else:
        moved = raw[:0]
    positions = np.where(keep, rank, raw).astype(np.int32)
    if len(moved):
        next_position = int(keep.sum())
    else:
        next_position = n
    old = moved.astype(np.int32)
    new = rank[moved].astype(np.int32)
    return keep, positions, moved.astype(np.int32), old, new, next_position
