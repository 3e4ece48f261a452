"""Request-local KV page ownership across prefill forwards: the native
plan, advance and bind of the multi-forward occurrence planner.

The reference's ``OccurrenceState`` (``akv/system/sglang/srt/context_system/
occurrence.py:470-920``) keeps the radix-cache bookkeeping -- matched
prefixes (``from_match``, ``reuse_match_gap``), which terminal versions a
forward publishes (``prefill_terminal_keep``), publication and Drop of
borrowed owners, SWA residency helpers and the release of private pages
(``free_context_slots``, ``ContextPrefillCompletion``).  It stays the caller
here.  What this module replaces is the hot part of a forward
(``occurrence.py:341-466`` plan, ``:632-767`` advance and terminal slots,
``:269-338`` bind): the host decisions run in C++ (``akv_plan_ownership`` /
``akv_advance_ownership``) on CPU metadata, and slot values never leave the
device: every list of slots a step produces is one segment of a single
batched gather launch (``akv_gather_slots``) fed by one host-to-device
copy, and :func:`advance_batch` binds a whole batch of requests with one
copy and one launch.  Names, fields and ``ValueError`` messages of the
calls kept here are the reference's.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .ops import _on_device, current_stream_handle

_SLOT_DTYPES = {torch.int32: _lib.AKV_I32, torch.int64: _lib.AKV_I64}


def _ptr(a):
    """Host pointer of a contiguous numpy array (None when empty)."""
    return ctypes.c_void_p(a.ctypes.data) if a.size else None


def _np(t, dtype):
    return np.ascontiguousarray(t.numpy() if isinstance(t, torch.Tensor) else t, dtype=dtype)


# ---------------------------------------------------------------------------
# Batched owner-row -> slot gathers (one upload, one launch).


class _Gather:
    """Segments of owner rows resolved against per-request slot pieces."""

    def __init__(self, device, dtype):
        self.device, self.dtype = device, dtype
        self.requests = []  # [(piece0, piece1, piece2)]
        self.wide, self.narrow = [], []  # [(request, rows)]

    def request(self, *pieces):
        pieces = [p for p in pieces] + [None] * (3 - len(pieces))
        for p in pieces:
            if p is not None and (p.dtype != self.dtype or p.device != self.device or p.ndim != 1):
                raise ValueError("Occurrence slot buffers do not match the ownership plan")
        self.requests.append(tuple(p if p is None or p.is_contiguous() else p.contiguous() for p in pieces))
        return len(self.requests) - 1

    def add(self, request, rows, narrow=False):
        (self.narrow if narrow else self.wide).append((request, np.asarray(rows, dtype=np.int64)))
        return (len(self.narrow) - 1) if narrow else (len(self.wide) - 1)

    def run(self, extra_i32=()):
        """Returns (wide slices, narrow slices, extra int32 slices)."""
        segments = self.wide + self.narrow
        lengths = np.array([len(r) for _, r in segments], dtype=np.int64)
        offsets = np.concatenate(([0], np.cumsum(lengths)))
        total = int(offsets[-1])
        wide_total = int(offsets[len(self.wide)])
        sources = np.zeros((len(self.requests), 6), dtype=np.int64)
        for b, pieces in enumerate(self.requests):
            for k, p in enumerate(pieces):
                if p is not None and p.numel():
                    sources[b, 2 * k] = p.data_ptr()
                    sources[b, 2 * k + 1] = p.numel()
        extra = [np.ascontiguousarray(e, dtype=np.int32).reshape(-1) for e in extra_i32]
        extra_words = [(len(e) + 1) // 2 for e in extra]
        parts = [sources.reshape(-1), offsets, np.array([b for b, _ in segments], dtype=np.int64)]
        parts += [r for _, r in segments]
        for e, words in zip(extra, extra_words):
            padded = np.zeros(2 * words, dtype=np.int32)
            padded[: len(e)] = e
            parts.append(padded.view(np.int64))
        host = np.concatenate(parts) if parts else np.zeros(0, np.int64)
        buf = torch.from_numpy(host).to(self.device, non_blocking=True)
        at = 0

        def take(k):
            nonlocal at
            view = buf[at : at + k]
            at += k
            return view

        d_sources, d_offsets, d_requests = take(sources.size), take(len(offsets)), take(len(segments))
        d_rows = take(total)
        extra_views = [take(w).view(torch.int32)[: len(e)] for e, w in zip(extra, extra_words)]
        out_wide = torch.empty(wide_total, dtype=self.dtype, device=self.device)
        out_narrow = torch.empty(total - wide_total, dtype=torch.int32, device=self.device)
        if total:
            lib = _lib.load()
            with _on_device(self.device):
                rc = lib.akv_gather_slots(
                    _SLOT_DTYPES[self.dtype], d_sources.data_ptr(), len(self.requests), len(segments),
                    d_offsets.data_ptr(),
                    d_requests.data_ptr(), d_rows.data_ptr(), total, wide_total,
                    out_wide.data_ptr() if wide_total else None,
                    out_narrow.data_ptr() if total > wide_total else None, current_stream_handle(self.device))
            _lib.check(rc, "akv_gather_slots")
        wide = [out_wide[offsets[i] : offsets[i + 1]] for i in range(len(self.wide))]
        narrow = [out_narrow[offsets[i] - wide_total : offsets[i + 1] - wide_total]
                  for i in range(len(self.wide), len(segments))]
        return wide, narrow, extra_views


def _gather_one(slots, rows):
    """slots[rows] (rows >= 0; -1 gives -1) with one launch."""
    g = _Gather(slots.device, slots.dtype)
    b = g.request(slots)
    g.add(b, rows)
    return g.run()[0][0]


# ---------------------------------------------------------------------------
# Plan.


@dataclass(frozen=True)
class OccurrenceMaterialization:
    """CPU ownership decision of one forward, made before the allocation
    (``occurrence.py:269-338``).  Source rows address canonical slots
    ``[0, n)`` first, then terminal slots ``[n, 2n)``; -1 = fresh or unbound."""

    source_rows: torch.Tensor
    allocated_occurrences: torch.Tensor
    copy_occurrences: torch.Tensor
    copy_source_rows: torch.Tensor
    copy_position_pairs: torch.Tensor
    terminal_occurrences: torch.Tensor
    read_cached: torch.Tensor
    repositioned_cached: torch.Tensor

    @property
    def extra_page_count(self) -> int:
        return len(self.allocated_occurrences)

    def bind(self, canonical_slots, terminal_slots, allocated_slots):
        """Device slots of every occurrence plus the copy lists, without a
        device-to-host read: one upload, one gather launch."""
        n = len(self.read_cached)
        if (
            canonical_slots.ndim != 1
            or terminal_slots.ndim != 1
            or allocated_slots.ndim != 1
            or any(v.dtype not in (torch.int32, torch.int64)
                   for v in (canonical_slots, terminal_slots, allocated_slots))
            or canonical_slots.dtype != terminal_slots.dtype
            or canonical_slots.dtype != allocated_slots.dtype
            or len(canonical_slots) != n
            or len(terminal_slots) != n
            or len(allocated_slots) != self.extra_page_count
            or canonical_slots.device != terminal_slots.device
            or canonical_slots.device != allocated_slots.device
        ):
            raise ValueError("Occurrence slot buffers do not match the ownership plan")
        rows = self.source_rows.numpy().copy()
        allocated = self.allocated_occurrences.numpy()
        rows[allocated] = 2 * n + np.arange(len(allocated))
        g = _Gather(canonical_slots.device, canonical_slots.dtype)
        b = g.request(canonical_slots, terminal_slots, allocated_slots)
        g.add(b, rows)
        g.add(b, self.copy_source_rows.numpy(), narrow=True)
        g.add(b, rows[self.copy_occurrences.numpy()], narrow=True)
        (slots,), (src, dst), (pairs,) = g.run((self.copy_position_pairs.numpy(),))
        return slots, src, dst, pairs.view(-1, 2)


def plan_occurrence_materialization(
    window,
    canonical_positions,
    canonical_present,
    canonical_owned,
    terminal_present,
    terminal_keep,
    *,
    query_start: int,
    query_end: int,
    exact_prefix_len: int,
) -> OccurrenceMaterialization:
    """Minimum occurrence allocations under explicit ownership
    (``occurrence.py:341-466``): reuse a terminal owner at the same
    position, else a canonical owner at the same position unless it is a
    borrowed page past the exact prefix that this forward publishes; copy
    the rest from the canonical owner (else the terminal one)."""
    n = len(window.birth_occurrences)
    if not 0 <= exact_prefix_len <= query_start < query_end <= n:
        raise ValueError("Invalid occurrence ownership/query boundaries")
    for value, size, dtype in (
        (canonical_positions, query_start, torch.int32),
        (canonical_present, query_start, torch.bool),
        (canonical_owned, query_start, torch.bool),
        (terminal_present, query_start, torch.bool),
        (terminal_keep, query_end, torch.bool),
    ):
        if value.device.type != "cpu" or value.dtype != dtype or value.shape != (size,):
            raise ValueError("Occurrence ownership must use aligned CPU metadata")
    if int(window.segment_query_starts[0]) != query_start or int(window.segment_query_ends[-1]) != query_end:
        raise ValueError("Occurrence ownership does not cover the planned queries")
    raw = _np(window.occurrence_raw_tokens, np.int32)
    pos = _np(window.occurrence_positions, np.int32)
    term = _np(window.terminal_occurrences, np.int32)
    keys = _np(window.segment_key_occurrences, np.int32)
    count = len(raw)
    u8 = lambda t: _np(t, np.bool_).view(np.uint8)
    cpos, cpres, cown, tpres, keep = (_np(canonical_positions, np.int32), u8(canonical_present),
                                      u8(canonical_owned), u8(terminal_present), u8(terminal_keep))
    source_rows = np.empty(count, dtype=np.int64)
    allocated = np.empty(max(count, 1), dtype=np.int64)
    copy_rows = np.empty(max(count, 1), dtype=np.int64)
    pairs = np.empty((max(count, 1), 2), dtype=np.int32)
    selected = np.empty(query_end, dtype=np.int64)
    read_cached = np.empty(n, dtype=np.bool_)
    rotated = np.empty(n, dtype=np.bool_)
    a = np.zeros(1, dtype=np.int64)
    rc = _lib.load().akv_plan_ownership(
        n, query_start, query_end, exact_prefix_len, count, _ptr(raw), _ptr(pos), _ptr(term), len(keys), _ptr(keys),
        _ptr(cpos), _ptr(cpres), _ptr(cown), _ptr(tpres), _ptr(keep), _ptr(source_rows), _ptr(allocated),
        _ptr(copy_rows), _ptr(pairs), _ptr(selected), _ptr(read_cached.view(np.uint8)),
        _ptr(rotated.view(np.uint8)), _ptr(a))
    _lib.check(rc, "akv_plan_ownership")
    k = int(a[0])
    return OccurrenceMaterialization(
        torch.from_numpy(source_rows),
        torch.from_numpy(allocated[:k].copy()),
        torch.from_numpy(allocated[:k].copy()),
        torch.from_numpy(copy_rows[:k].copy()),
        torch.from_numpy(pairs[:k].copy()),
        torch.from_numpy(selected),
        torch.from_numpy(read_cached),
        torch.from_numpy(rotated),
    )


# ---------------------------------------------------------------------------
# State.


@dataclass(frozen=True)
class OccurrenceAdvance:
    """Result of binding one forward (``occurrence.py:922-933``)."""

    state: "OccurrenceState"
    occurrence_slots: torch.Tensor
    copy_source_slots: torch.Tensor
    copy_destination_slots: torch.Tensor
    copy_position_pairs: torch.Tensor
    # released exactly once, after the forward's completion event
    retired_slots: torch.Tensor
    # fresh SWA peers with no valid source: release their SWA mapping only
    unused_swa_slots: torch.Tensor | None = None
    retired_swa_resident: torch.Tensor | None = None


@dataclass(frozen=True)
class OccurrenceState:
    """Request-local page ownership between prefill forwards: the fields of
    the reference's ``OccurrenceState`` (``occurrence.py:470-490``).  CPU
    rows index ``slots`` (device); a row is a page the request owns
    (``owned``) or borrows from the cache.  The reference's state methods
    that build and edit these fields outside a forward (matches, publication,
    Drop of borrowed owners) stay the reference's."""

    slots: torch.Tensor
    owned: torch.Tensor
    canonical_rows: torch.Tensor
    terminal_rows: torch.Tensor
    canonical_positions: torch.Tensor
    exact_prefix_len: int
    swa_resident: torch.Tensor | None = None

    @classmethod
    def empty(cls, device, slot_dtype=torch.int64, *, track_swa=False):
        """The state of a request with no matched prefix: nothing owned,
        nothing canonical, no terminal versions."""
        if slot_dtype not in _SLOT_DTYPES:
            raise ValueError("Occurrence slots must be int32 or int64")
        none64 = torch.empty(0, dtype=torch.int64)
        return cls(torch.empty(0, dtype=slot_dtype, device=device), torch.empty(0, dtype=torch.bool), none64,
                   none64.clone(), torch.empty(0, dtype=torch.int32), 0,
                   torch.empty(0, dtype=torch.bool) if track_swa else None)

    def plan(self, window, terminal_keep):
        """The forward's ownership plan (``akv_plan_ownership``) over this
        state's rows; ``terminal_keep`` is the caller's choice of the raw
        tokens whose terminal versions the forward publishes."""
        start = len(self.canonical_rows)
        canonical = self.canonical_rows.numpy()
        present = canonical >= 0
        owned = np.zeros(start, dtype=np.bool_)
        owned[present] = self.owned.numpy()[canonical[present]]
        return plan_occurrence_materialization(
            window, self.canonical_positions, torch.from_numpy(present), torch.from_numpy(owned),
            self.terminal_rows >= 0, terminal_keep, query_start=start,
            query_end=int(window.segment_query_ends[-1]), exact_prefix_len=self.exact_prefix_len)

    def advance(self, window, plan, query_slots, extra_slots, visible_until):
        """Bind one admitted forward (``occurrence.py:632-755``); see
        :func:`advance_batch` for a batch in one launch."""
        return advance_batch([(self, window, plan, query_slots, extra_slots, visible_until)])[0][0]

    def terminal_slots(self):
        """Raw-order final-position slots, -1 for holes (``:757-767``)."""
        return _gather_one(self.slots, self.terminal_rows.numpy())


# ---------------------------------------------------------------------------
# Batched advance.


@dataclass(frozen=True)
class BatchAdvance:
    """Concatenated lists of a batch's forwards (the prefill input of the
    reference's ``_prepare_context_occurrences``, ``sglang.patch:3174-3180``)."""

    occurrence_slots: torch.Tensor
    copy_source_slots: torch.Tensor
    copy_destination_slots: torch.Tensor
    copy_position_pairs: torch.Tensor


def advance_rows(state, window, plan, query_count, extra_count, visible_until):
    """Host half of an advance (``akv_advance_ownership``): owner-row lists
    over the request's slot sequence old ++ query ++ extra, the successor's
    CPU metadata and the list lengths.  No device work."""
    n = len(window.birth_occurrences)
    start, end = len(state.canonical_rows), len(plan.terminal_occurrences)
    old = len(state.slots)
    q, a = int(query_count), int(extra_count)
    cap = max(old + q + a, 1)
    count = len(window.occurrence_raw_tokens)
    track = state.swa_resident is not None
    o = dict(
        occ=np.empty(count, np.int64), src=np.empty(max(a, 1), np.int64), dst=np.empty(max(a, 1), np.int64),
        keep=np.empty(cap, np.int64), retired=np.empty(cap, np.int64), unused=np.empty(max(a, 1), np.int64),
        owned=np.empty(cap, np.uint8), canonical=np.empty(end, np.int64), terminal=np.empty(end, np.int64),
        positions=np.empty(end, np.int32), swa=np.empty(cap, np.uint8), retired_swa=np.empty(cap, np.uint8),
        counts=np.zeros(3, np.int64),
    )
    owned = _np(state.owned, np.bool_).view(np.uint8)
    swa = _np(state.swa_resident, np.bool_).view(np.uint8) if track else np.zeros(0, np.uint8)
    rc = _lib.load().akv_advance_ownership(
        n, start, end, old, q, a, _ptr(owned), _ptr(_np(state.canonical_rows, np.int64)),
        _ptr(_np(state.terminal_rows, np.int64)), _ptr(_np(state.canonical_positions, np.int32)), int(track),
        _ptr(swa), count, _ptr(_np(window.occurrence_positions, np.int32)),
        _ptr(_np(window.terminal_occurrences, np.int32)), _ptr(_np(plan.source_rows, np.int64)),
        _ptr(_np(plan.allocated_occurrences, np.int64)), _ptr(_np(plan.copy_source_rows, np.int64)),
        _ptr(_np(plan.terminal_occurrences, np.int64)), _ptr(_np(visible_until, np.int32)),
        *(_ptr(o[k]) for k in ("occ", "src", "dst", "keep", "retired", "unused", "owned", "canonical", "terminal",
                               "positions", "swa", "retired_swa", "counts")))
    _lib.check(rc, "akv_advance_ownership")
    kept, retired, unused = (int(x) for x in o["counts"])
    return dict(
        occurrence=o["occ"], copy_source=o["src"][:a], copy_destination=o["dst"][:a], successor=o["keep"][:kept],
        retired=o["retired"][:retired], unused_swa=o["unused"][:unused] if track else None,
        owned=o["owned"][:kept].astype(np.bool_), canonical_rows=o["canonical"], terminal_rows=o["terminal"],
        canonical_positions=o["positions"], swa_resident=o["swa"][:kept].astype(np.bool_) if track else None,
        retired_swa_resident=o["retired_swa"][:retired].astype(np.bool_) if track else None,
    )


def advance_batch(steps):
    """Bind the forwards of a batch: ``steps`` = [(state, window, plan,
    query_slots, extra_slots, visible_until)].  Host index work per request
    in C++, then one upload and one gather launch for every slot list of
    every request.  Returns ([OccurrenceAdvance], BatchAdvance)."""
    if not steps:
        raise ValueError("advance_batch needs at least one forward")
    device = steps[0][3].device
    dtype = steps[0][3].dtype
    if dtype not in _SLOT_DTYPES:
        raise ValueError("Context admission does not cover the selected window")
    g = _Gather(device, dtype)
    pending = []
    for state, window, plan, query_slots, extra_slots, visible_until in steps:
        n = len(window.birth_occurrences)
        start, end = len(state.canonical_rows), len(plan.terminal_occurrences)
        if (
            query_slots.ndim != 1
            or extra_slots.ndim != 1
            or len(query_slots) != end - start
            or len(extra_slots) != plan.extra_page_count
            or query_slots.dtype != state.slots.dtype
            or extra_slots.dtype != state.slots.dtype
            or (len(state.slots) and query_slots.device != state.slots.device)
            or extra_slots.device != query_slots.device
            or visible_until.device.type != "cpu"
            or visible_until.dtype != torch.int32
            or visible_until.shape != (n,)
        ):
            raise ValueError("Context admission does not cover the selected window")
        if query_slots.device != device or query_slots.dtype != dtype:
            raise ValueError("A batch's slots must share one device and dtype")
        r = advance_rows(state, window, plan, len(query_slots), len(extra_slots), visible_until)
        b = g.request(state.slots if len(state.slots) else None, query_slots, extra_slots)
        seg = dict(occ=g.add(b, r["occurrence"]), keep=g.add(b, r["successor"]), retired=g.add(b, r["retired"]),
                   unused=g.add(b, r["unused_swa"]) if r["unused_swa"] is not None else None,
                   src=g.add(b, r["copy_source"], narrow=True), dst=g.add(b, r["copy_destination"], narrow=True))
        pending.append((state, plan, r, seg))
    wide, narrow, pairs = g.run([p[1].copy_position_pairs.numpy().reshape(-1) for p in pending])
    results = []
    for (state, plan, r, seg), pair in zip(pending, pairs):
        track = r["swa_resident"] is not None
        successor = OccurrenceState(
            wide[seg["keep"]], torch.from_numpy(r["owned"]), torch.from_numpy(r["canonical_rows"]),
            torch.from_numpy(r["terminal_rows"]), torch.from_numpy(r["canonical_positions"]), state.exact_prefix_len,
            torch.from_numpy(r["swa_resident"]) if track else None)
        results.append(OccurrenceAdvance(
            successor, wide[seg["occ"]], narrow[seg["src"]], narrow[seg["dst"]], pair.view(-1, 2),
            wide[seg["retired"]], wide[seg["unused"]] if track else None,
            torch.from_numpy(r["retired_swa_resident"]) if track else None))
    cat = lambda ts: torch.cat(ts) if len(ts) > 1 else ts[0]
    batch = BatchAdvance(cat([x.occurrence_slots for x in results]), cat([x.copy_source_slots for x in results]),
                         cat([x.copy_destination_slots for x in results]),
                         cat([x.copy_position_pairs for x in results]))
    return results, batch
