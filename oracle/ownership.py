"""CPU restatement of request-local KV page ownership across prefill
forwards -- TEST INFRASTRUCTURE ONLY (see the package docstring).

A request's prompt may be computed in several forwards (chunked prefill, a
matched prefix borrowed from the radix cache, recovery gaps).  Between
forwards a state records, for every raw token computed so far, which owner
row holds its *canonical* version (the one later queries read) and which
holds its *terminal* version (final position, published to the cache).
Each forward plans which occurrence versions need a page, reuses the ones
that already exist at the right position, allocates the rest (filled by
copy + RoPE rotation), and retires the private pages nothing needs any more.

Restates ``akv/system/sglang/srt/context_system/occurrence.py``:

``plan``                  ``plan_occurrence_materialization`` (:341-466)
``State.from_match``      ``OccurrenceState.from_match`` (:491-526)
``State.reuse_match_gap`` (:528-586)
``State.prefill_terminal_keep`` (:588-612)
``State.plan``            (:614-630)
``State.advance``         (:632-755) -- returns the successor and the
                          gathered slot lists of ``OccurrenceAdvance`` (:922-933)
``State.terminal_slots``  (:757-767)
``State.publish``         (:769-821)
``State.drop_borrowed_raw`` (:823-864)
``State.terminal_swa_residency``, ``private_slots``,
``nonterminal_private_residency``, ``nonterminal_private_slots`` (:866-920)

Slots are numpy int64 here (device tensors in the reference); every index
decision is the same.

Pinned by (``tests/test_oracle_ownership.py``): a symbolic execution of the
KV pool (each slot holds a ``(raw token, position)`` version tag, queries
write their birth versions, copies move a tag and check the source) over
random multi-stage programs computed in 1-4 forwards with borrowed prefixes,
holes and recovery gaps -- every read occurrence finds its version, every
published terminal slot holds the final version, no live or borrowed page
is retired, every private page is retired exactly once over a request's
life; at ``query_start = 0`` the plan and advance equal the final-forward
restatement in ``oracle/occurrence.py`` (itself pinned by a closed form);
the reuse / allocation / retirement choices the symbolic model leaves open
are pinned by golden vectors written from the reference module
(``tests/golden/ownership_vectors.npz``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


def plan(window, canonical_positions, canonical_present, canonical_owned, terminal_present, terminal_keep, *,
         query_start, query_end, exact_prefix_len):
    """Which occurrences need a page, which reuse an existing owner row, and
    the copies that fill the allocated ones.

    Owner rows address ``canonical[0:n] ++ terminal[0:n]`` of the raw tokens:
    row ``r`` = canonical version of raw ``r``, row ``n + r`` = its terminal
    version.  Query tokens of this forward are present and owned at their
    birth position.
    """
    raw = np.asarray(window["raw"], dtype=np.int64)
    pos = np.asarray(window["pos"], dtype=np.int64)
    birth = np.asarray(window["birth"], dtype=np.int64)
    term = np.asarray(window["terminal"], dtype=np.int64)
    n = len(birth)
    if not 0 <= exact_prefix_len <= query_start < query_end <= n:
        raise ValueError("Invalid occurrence ownership/query boundaries")
    count = len(raw)
    have = np.zeros(n, dtype=bool)
    mine = np.zeros(n, dtype=bool)
    have[:query_start] = canonical_present
    mine[:query_start] = canonical_owned
    have[query_start:query_end] = True
    mine[query_start:query_end] = True
    cpos = pos[birth].copy()
    cpos[:query_start] = canonical_positions
    tlive = np.zeros(n, dtype=bool)
    tlive[:query_start] = terminal_present
    tpos = pos[term]

    read = np.zeros(count, dtype=bool)
    read[np.asarray(window["keys"], dtype=np.int64)] = True
    need = read.copy()
    need[birth[query_start:query_end]] = True
    published_raw = np.flatnonzero(np.asarray(terminal_keep, dtype=bool))
    published = term[published_raw]
    need[published] = True
    publishing = np.zeros(count, dtype=bool)
    publishing[published] = True

    ids = np.flatnonzero(need)
    r, p = raw[ids], pos[ids]
    at_terminal = tlive[r] & (tpos[r] == p)
    at_canonical = have[r] & (cpos[r] == p)
    # a borrowed page past the exact prefix cannot become this version's
    # published owner, even at the same position
    must_own = publishing[ids] & (r >= exact_prefix_len) & ~mine[r] & ~at_terminal
    reuse = at_terminal | (at_canonical & ~must_own)
    source_rows = np.full(count, -1, dtype=np.int64)
    source_rows[ids[reuse]] = np.where(at_terminal, n + r, r)[reuse]

    allocated = ids[~reuse]
    ar = raw[allocated]
    from_terminal = ~have[ar] & tlive[ar]
    lost = ~have[ar] & ~tlive[ar]
    if lost.any():
        raise ValueError("Occurrence recovery required for raw tokens " + repr(np.unique(ar[lost]).tolist()))
    copy_rows = np.where(from_terminal, n + ar, ar)
    old = np.where(from_terminal, tpos[ar], cpos[ar])
    pairs = np.stack((old, pos[allocated]), axis=1).astype(np.int32)

    terminal_occ = np.full(query_end, -1, dtype=np.int64)
    terminal_occ[published_raw] = published
    read_raw = raw[read]
    read_cached = np.zeros(n, dtype=bool)
    read_cached[read_raw[read_raw < query_start]] = True
    rotated = read[ids] & (p != cpos[r]) & (r < query_start)
    repositioned_cached = np.zeros(n, dtype=bool)
    repositioned_cached[r[rotated]] = True
    return {
        "source_rows": source_rows,
        "allocated": allocated,
        "copy_occurrences": allocated.copy(),
        "copy_source_rows": copy_rows,
        "pairs": pairs,
        "terminal_occurrences": terminal_occ,
        "read_cached": read_cached,
        "repositioned_cached": repositioned_cached,
        "extra_page_count": len(allocated),
    }


@dataclass
class Advance:
    state: "State"
    occurrence_slots: np.ndarray
    copy_source_slots: np.ndarray
    copy_destination_slots: np.ndarray
    copy_position_pairs: np.ndarray
    retired_slots: np.ndarray
    unused_swa_slots: np.ndarray | None = None
    retired_swa_resident: np.ndarray | None = None
    # owner-row form of the same lists (indices into old ++ query ++ extra)
    rows: dict = field(default_factory=dict)


@dataclass
class State:
    slots: np.ndarray
    owned: np.ndarray
    canonical_rows: np.ndarray
    terminal_rows: np.ndarray
    canonical_positions: np.ndarray
    exact_prefix_len: int
    swa_resident: np.ndarray | None = None

    @classmethod
    def from_match(cls, slots, positions, *, exact_prefix_len, resident=None, swa_resident=None):
        slots = np.asarray(slots, dtype=np.int64)
        positions = np.asarray(positions, dtype=np.int32)
        if positions.shape != slots.shape or not 0 <= exact_prefix_len <= len(slots):
            raise ValueError("Invalid Context match ownership metadata")
        rows = np.arange(len(slots), dtype=np.int64)
        if resident is not None:
            rows[~np.asarray(resident, dtype=bool)] = -1
        return cls(slots.copy(), np.zeros(len(slots), dtype=bool), rows, np.full(len(slots), -1, dtype=np.int64),
                   positions.copy(), int(exact_prefix_len),
                   None if swa_resident is None else np.asarray(swa_resident, dtype=bool).copy())

    @property
    def start(self):
        return len(self.canonical_rows)

    def reuse_match_gap(self, matched_slots, matched_positions, resident, end, *, exact_prefix_len,
                        swa_resident=None):
        """Borrow matched pages for the resident gap ``[start, end)``."""
        start = self.start
        matched_slots = np.asarray(matched_slots, dtype=np.int64)
        if not start <= end <= len(matched_slots) or not self.exact_prefix_len <= exact_prefix_len <= len(
                matched_slots):
            raise ValueError("Invalid matched gap ownership metadata")
        if (self.swa_resident is None) != (swa_resident is None):
            raise ValueError("Context matched gap must preserve SWA residency metadata")
        if end == start:
            return self
        k = end - start
        rows = np.arange(len(self.slots), len(self.slots) + k, dtype=np.int64)
        rows[~np.asarray(resident, dtype=bool)[start:end]] = -1
        return State(
            np.concatenate((self.slots, matched_slots[start:end])),
            np.concatenate((self.owned, np.zeros(k, dtype=bool))),
            np.concatenate((self.canonical_rows, rows)),
            np.concatenate((self.terminal_rows, np.full(k, -1, dtype=np.int64))),
            np.concatenate((self.canonical_positions, np.asarray(matched_positions, dtype=np.int32)[start:end])),
            min(end, exact_prefix_len),
            None if swa_resident is None else np.concatenate(
                (self.swa_resident, np.asarray(swa_resident, dtype=bool)[start:end])),
        )

    def prefill_terminal_keep(self, layout, query_end):
        """Raw tokens whose terminal version this forward publishes."""
        start = self.start
        keep = np.asarray(layout.keep_mask[:query_end], dtype=bool).copy()
        keep[:start] &= (self.canonical_rows >= 0) | (self.terminal_rows >= 0)
        if query_end < len(layout.positions):
            # before the final forward only versions already at their final
            # position are published
            final = np.asarray(layout.positions[:query_end])
            ready = np.asarray(layout.birth_positions[:query_end]) == final
            ready[:start] = (self.canonical_positions == final[:start]) | (self.terminal_rows >= 0)
            keep &= ready
        return keep

    def plan(self, window, terminal_keep):
        start = self.start
        present = self.canonical_rows >= 0
        owned = np.zeros(start, dtype=bool)
        owned[present] = self.owned[self.canonical_rows[present]]
        return plan(window, self.canonical_positions, present, owned, self.terminal_rows >= 0, terminal_keep,
                    query_start=start, query_end=int(window["ends"][-1]), exact_prefix_len=self.exact_prefix_len)

    def advance(self, window, p, query_slots, extra_slots, visible_until):
        """Bind this forward's birth and fresh slots; successor + slot lists."""
        n = len(window["birth"])
        start, end = self.start, len(p["terminal_occurrences"])
        query_slots = np.asarray(query_slots, dtype=np.int64)
        extra_slots = np.asarray(extra_slots, dtype=np.int64)
        if len(query_slots) != end - start or len(extra_slots) != p["extra_page_count"] or len(visible_until) != n:
            raise ValueError("Context admission does not cover the selected window")
        old = len(self.slots)
        q, a = len(query_slots), len(extra_slots)
        everything = np.concatenate((self.slots, query_slots, extra_slots))
        owned = np.concatenate((self.owned, np.ones(q + a, dtype=bool)))
        canonical = np.full(n, -1, dtype=np.int64)
        canonical[:start] = self.canonical_rows
        canonical[start:end] = np.arange(old, old + q)
        terminal = np.full(n, -1, dtype=np.int64)
        terminal[:start] = self.terminal_rows
        by_row = np.concatenate((canonical, terminal))

        src = p["source_rows"]
        occ = np.full(len(src), -1, dtype=np.int64)
        hit = src >= 0
        occ[hit] = by_row[src[hit]]
        if np.any(occ[hit] < 0):
            raise ValueError("Context ownership plan references a missing source")
        occ[p["allocated"]] = np.arange(old + q, old + q + a)
        copy_from = by_row[p["copy_source_rows"]]
        if np.any(copy_from < 0):
            raise ValueError("Context copy references a missing canonical source")
        copy_to = occ[p["copy_occurrences"]]

        swa = None
        unused = np.zeros(0, dtype=np.int64)
        if self.swa_resident is not None:
            swa = np.concatenate((self.swa_resident, np.ones(q + a, dtype=bool)))
            swa[copy_to] = swa[copy_from]
            unused = copy_to[~swa[copy_to]]

        chosen = p["terminal_occurrences"]
        kept = chosen >= 0
        new_terminal = np.full(end, -1, dtype=np.int64)
        new_terminal[kept] = occ[chosen[kept]]
        wpos = np.asarray(window["pos"], dtype=np.int64)
        positions = wpos[np.asarray(window["birth"])[:end]].astype(np.int32)
        positions[:start] = self.canonical_positions
        final = wpos[np.asarray(window["terminal"])[:end]]
        new_canonical = canonical[:end].copy()
        # a same-position terminal copy is bit-identical: later reads use it
        same = kept & (positions == final)
        new_canonical[same] = new_terminal[same]
        if end == n:
            new_canonical[:] = -1
        else:
            new_canonical[np.asarray(visible_until)[:end] <= end] = -1

        live = np.zeros(len(everything), dtype=bool)
        live[new_canonical[new_canonical >= 0]] = True
        live[new_terminal[kept]] = True
        kept_rows = np.flatnonzero(live)
        retired = np.flatnonzero(owned & ~live)
        remap = np.full(len(everything), -1, dtype=np.int64)
        remap[kept_rows] = np.arange(len(kept_rows))
        succ_canonical = np.where(new_canonical >= 0, remap[np.maximum(new_canonical, 0)], -1)
        succ_terminal = np.where(kept, remap[np.maximum(new_terminal, 0)], -1)
        successor = State(everything[kept_rows], owned[kept_rows], succ_canonical, succ_terminal, positions,
                          self.exact_prefix_len, None if swa is None else swa[kept_rows])
        rows = {
            "occurrence": np.maximum(occ, 0),
            "copy_source": copy_from,
            "copy_destination": copy_to,
            "successor": kept_rows,
            "retired": retired,
            "unused_swa": unused,
        }
        return Advance(
            successor,
            everything[rows["occurrence"]],
            everything[copy_from].astype(np.int32),
            everything[copy_to].astype(np.int32),
            p["pairs"].reshape(-1, 2).astype(np.int32),
            everything[retired],
            everything[unused] if swa is not None else None,
            swa[retired] if swa is not None else None,
            rows,
        )

    def terminal_slots(self):
        out = np.full(len(self.terminal_rows), -1, dtype=np.int64)
        present = self.terminal_rows >= 0
        out[present] = self.slots[self.terminal_rows[present]]
        return out

    def publish(self, matched_terminal_slots, *, cache_len=None, swa_resident=None):
        """Hand the published terminal versions to the cache's owners."""
        rows = self.terminal_rows
        matched = np.asarray(matched_terminal_slots, dtype=np.int64)
        if matched.shape != rows.shape:
            raise ValueError("Context publication must cover the raw terminal table")
        cache_len = len(rows) if cache_len is None else cache_len
        if not 0 <= cache_len <= len(rows):
            raise ValueError("Context cache publication length exceeds the raw table")
        present = np.flatnonzero(rows[:cache_len] >= 0)
        target = rows[present]
        if len(np.unique(target)) != len(target):
            raise ValueError("Distinct raw tokens cannot publish the same KV owner")
        slots = self.slots.copy()
        slots[target] = matched[present]
        owned = self.owned.copy()
        owned[target] = False
        swa = self.swa_resident
        if swa_resident is not None:
            if swa is None or np.asarray(swa_resident).shape != rows.shape:
                raise ValueError("Context publication SWA metadata must cover the raw table")
            swa = swa.copy()
            swa[target] = np.asarray(swa_resident, dtype=bool)[present]
        return State(slots, owned, self.canonical_rows, self.terminal_rows, self.canonical_positions,
                     self.exact_prefix_len, swa)

    def drop_borrowed_raw(self, dropped):
        """Forget borrowed (unowned) versions of dropped raw tokens."""
        dropped = np.asarray(dropped, dtype=bool)
        if dropped.shape != self.terminal_rows.shape:
            raise ValueError("Context Drop ownership mask must cover the raw state")
        canonical = self.canonical_rows.copy()
        terminal = self.terminal_rows.copy()
        changed = False
        for rows in (canonical, terminal):
            hit = np.flatnonzero(dropped & (rows >= 0))
            hit = hit[~self.owned[rows[hit]]]
            if len(hit):
                rows[hit] = -1
                changed = True
        if not changed:
            return self
        live = self.owned.copy()
        live[canonical[canonical >= 0]] = True
        live[terminal[terminal >= 0]] = True
        kept_rows = np.flatnonzero(live)
        remap = np.full(len(live), -1, dtype=np.int64)
        remap[kept_rows] = np.arange(len(kept_rows))
        for rows in (canonical, terminal):
            rows[rows >= 0] = remap[rows[rows >= 0]]
        return State(self.slots[kept_rows], self.owned[kept_rows], canonical, terminal, self.canonical_positions,
                     self.exact_prefix_len, None if self.swa_resident is None else self.swa_resident[kept_rows])

    def terminal_swa_residency(self):
        if self.swa_resident is None:
            return None
        out = np.zeros(len(self.terminal_rows), dtype=bool)
        present = self.terminal_rows >= 0
        out[present] = self.swa_resident[self.terminal_rows[present]]
        return out

    def private_slots(self):
        return self.slots[self.owned]

    def _nonterminal_private(self):
        chosen = self.owned.copy()
        chosen[self.terminal_rows[self.terminal_rows >= 0]] = False
        return chosen

    def nonterminal_private_residency(self):
        return None if self.swa_resident is None else self.swa_resident[self._nonterminal_private()]

    def nonterminal_private_slots(self):
        return self.slots[self._nonterminal_private()]
