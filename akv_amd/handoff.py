"""Page-size-one Context handoff between a prefill (P) and a decode (D) engine.

Mirror of ``akv/system/sglang/srt/disaggregation/context_transfer.py:20-283``
(``ContextTransferPlan``, ``transfer_plan``, ``prepare_decode_transfer_plan``,
``request_active_slots``, ``request_active_lengths``,
``select_missing_transfer``, ``ContextDecodeReuse``,
``allocate_context_destination``, ``materialize_decode_reuse``): same
arguments, results and messages.  Raw request coordinates stay intact while
the transfer and D's allocation cover only final active versions.  Requests,
pools and allocators are the engine's own objects, read through the
attributes the reference reads.  Device work: slot lists come from one
``akv_gather_slots`` launch each, K/V rows move with ``akv_copy_kv_rows``
(``akv_amd.transfer``; the single-node stand-in for the transport) and
reused pages at new positions are repositioned by
``ContextModelBinding.reposition_existing``.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np
import torch

from .binding import ContextModelBinding
from .request_rows import request_row
from .ownership import OccurrenceState, _Gather
from .page_table import ContextDecodeLayout


def _row_gather(row, raw):
    """row[raw] on the device (``raw`` host indices), one launch."""
    g = _Gather(row.device, row.dtype)
    g.add(g.request(row), np.asarray(raw, dtype=np.int64))
    return g.run()[0][0]


@dataclass(frozen=True)
class ContextTransferPlan:
    """Final active versions of a request and the identity both sides check."""

    decode: ContextDecodeLayout
    signature: tuple

    @classmethod
    def build(cls, program, device):
        # the full event identity, not just the final tokens and positions
        digest = hashlib.blake2b(digest_size=8)
        for value in (program.layout.records, program.layout.keep_mask, program.visible_until):
            digest.update(value.numpy().tobytes())
        signature = tuple(int(x) for x in np.frombuffer(digest.digest(), dtype="<i4"))
        return cls(ContextDecodeLayout.from_layout(program.layout, device), signature)

    @property
    def active_count(self):
        return len(self.decode.raw_indices)

    def swa_start(self, window):
        """First active version the first D query can see (a key at
        ``query_position - window`` is still inside the window)."""
        return int(np.searchsorted(self.decode.positions, self.decode.next_position - window))

    def slots(self, req, pool, *, window=None):
        start = self.swa_start(window) if window is not None else 0
        return _row_gather(request_row(pool, req.kv.req_pool_idx), self.decode.raw_indices[start:])

    def full_chunk(self, raw_start, raw_end, *, last_chunk, terminal_rows=None, owned=None):
        """Active versions of the completed raw range as (begin, end, cursor).

        One version is withheld until the final send (the transport infers
        completion from the cumulative page count); a non-final send stops
        at the first version whose terminal owner is missing or still
        private (a later publication may deduplicate it); the raw cursor
        never passes a withheld version.
        """
        begin, end = np.searchsorted(self.decode.raw_indices, (raw_start, raw_end))
        if terminal_rows is not None:
            raw = self.decode.raw_indices[begin:end]
            rows = terminal_rows.numpy()[raw]
            ready = rows >= 0
            if last_chunk:
                if not ready.all():
                    raise ValueError("Context final transfer has missing terminal KV")
            else:
                if owned is not None:
                    ready[ready] = ~owned.numpy()[rows[ready]]
                missing = np.flatnonzero(~ready)
                if len(missing):
                    end = int(begin) + int(missing[0])
        if not last_chunk:
            end = min(int(end), max(0, self.active_count - 1))
        cursor = raw_end
        if end < self.active_count:
            cursor = min(cursor, int(self.decode.raw_indices[end]))
        return int(begin), int(end), cursor

    def header(self):
        return (2, self.active_count, self.decode.next_position, *self.signature)


def transfer_plan(req, device):
    program = req.context_recompute_program or req.context_program
    current = getattr(req, "context_transfer_plan", None)
    if current is None or current.decode.prompt_length != len(program.layout.positions):
        current = ContextTransferPlan.build(program, device)
        req.context_transfer_plan = current
    return current


def prepare_decode_transfer_plan(req, device, raw_length):
    """Plan over the prompt plus the tokens generated so far."""
    base = len(req.origin_input_ids)
    if raw_length > base and (
        req.context_recompute_program is None
        or len(req.context_recompute_program.layout.positions) != raw_length
    ):
        req.context_recompute_program = req.context_program.with_generated(req.output_ids[: raw_length - base])
    return transfer_plan(req, device)


def request_active_slots(req, pool, raw_end, *, window=None):
    """Slots of the compacted active row (kept prompt versions, then the
    generated tail up to ``raw_end``) -- never a hole; one gather launch."""
    view = req.context_decode_layout
    if view is None:
        view = ContextDecodeLayout.from_layout(req.context_program.layout, pool.req_to_token.device)
    start = 0
    generated_start = view.prompt_length
    if window is not None:
        lower = view.next_position + raw_end - view.prompt_length - window
        start = int(np.searchsorted(view.positions, lower))
        generated_start += max(0, lower - view.next_position)
    raw = np.concatenate((view.raw_indices[start:].astype(np.int64),
                          np.arange(generated_start, raw_end, dtype=np.int64)))
    return _row_gather(request_row(pool, req.kv.req_pool_idx), raw)


def request_active_lengths(req, raw_end, window):
    """(full, window) active lengths from CPU metadata only."""
    view = req.context_decode_layout
    generated = max(0, raw_end - view.prompt_length)
    full = len(view.raw_indices) + generated
    lower = view.next_position + generated - window
    start = int(np.searchsorted(view.positions, lower))
    return full, len(view.raw_indices) - start + min(generated, window)


def select_missing_transfer(source, destination, reusable):
    """One peer's chunk without the pages it can reuse."""
    if source.shape != destination.shape or reusable.shape != source.shape:
        raise ValueError("Context transfer bitmap and page coordinates disagree")
    if reusable.dtype != np.bool_:
        raise ValueError("Context transfer reuse bitmap must be boolean")
    missing = ~reusable
    return source[missing], destination[missing]


@dataclass(frozen=True)
class ContextDecodeReuse:
    """D's own cache match projected onto the final active versions.

    A matched, resident version outside the SWA tail is reused; at a new
    position, or past the exact prefix, it gets a private page filled by a
    copy (two cache branches never share an owner), otherwise it is
    borrowed as is.
    """

    source_slots: torch.Tensor
    reusable: np.ndarray
    borrowed: np.ndarray
    copy_indices: np.ndarray
    position_pairs: torch.Tensor

    @classmethod
    def build(cls, req, plan, *, window=None):
        raw = plan.decode.raw_indices
        matched = len(req.prefix_indices)
        reusable = raw < matched
        resident = req.context_resident
        if resident is not None:
            reusable[reusable] &= resident.numpy()[raw[reusable]]
        if window is not None:
            # the SWA tail arrives as one payload into fresh owners
            reusable[plan.swa_start(window):] = False
        source = req.context_source_positions
        if source is None:
            source = torch.arange(matched, dtype=torch.int32)
        borrowed = reusable.copy()
        indices = np.flatnonzero(reusable)
        old = source.numpy()[raw[indices]]
        new = plan.decode.positions[indices]
        copy = (old != new) | (raw[indices] >= req.context_exact_prefix_len)
        borrowed[indices[copy]] = False
        return cls(req.prefix_indices, reusable, borrowed, indices[copy],
                   torch.from_numpy(np.stack((old[copy], new[copy]), axis=1).astype(np.int32)))

    @property
    def allocation_count(self):
        return len(self.borrowed) - int(self.borrowed.sum())


def allocate_context_destination(req, allocator, pool, *, window=None):
    """Allocate D's owners of the active versions (fresh, or borrowed from
    its own cache match), bind the request's ownership state and write its
    raw-order table row."""
    plan = transfer_plan(req, allocator.device)
    count = plan.active_count
    reuse = getattr(req, "context_decode_reuse", None)
    allocation_count = count if reuse is None else reuse.allocation_count
    if window is None:
        allocated = allocator.alloc(allocation_count)
        swa = None
    else:
        start = plan.swa_start(window)
        if reuse is not None and reuse.reusable[start:].any():
            raise ValueError("Context SWA transfer destinations must be private")
        allocated = allocator.alloc_context_swa_tail(allocation_count, count - start)
        swa = torch.arange(count) >= start
    if allocated is None:
        raise RuntimeError("Context PD destination allocation exceeds admitted capacity")
    slots = allocated
    owned = torch.ones(count, dtype=torch.bool)
    if reuse is not None:
        allocated = allocated.to(torch.int64)
        owned = torch.from_numpy(~reuse.borrowed)
        private_raw = plan.decode.raw_indices[~reuse.borrowed]
        if len(private_raw):
            # a freshly received version is private even on an exact hit
            req.context_exact_prefix_len = min(req.context_exact_prefix_len, int(private_raw[0]))
        # slot i = next fresh slot when private, else the matched source slot
        rows = np.empty(count, dtype=np.int64)
        private = ~reuse.borrowed
        rows[private] = np.arange(int(private.sum()))
        rows[reuse.borrowed] = len(allocated) + plan.decode.raw_indices[reuse.borrowed].astype(np.int64)
        g = _Gather(allocated.device, torch.int64)
        g.add(g.request(allocated, reuse.source_slots.to(torch.int64)), rows)
        slots = g.run()[0][0]
    rows = torch.full((plan.decode.prompt_length,), -1, dtype=torch.int64)
    rows[torch.from_numpy(plan.decode.raw_indices.astype(np.int64))] = torch.arange(count)
    program = req.context_recompute_program or req.context_program
    req.context_state = OccurrenceState(
        slots, owned, rows, rows.clone(), program.layout.positions,
        min(req.context_exact_prefix_len, plan.decode.prompt_length) if reuse is not None else 0, swa)
    req.context_decode_layout = plan.decode
    req.context_prefill_started = True
    req.context_cache_published = reuse is None
    terminal = req.context_state.terminal_slots()
    pool.write((req.kv.req_pool_idx, slice(0, len(terminal))), terminal)
    req.kv.kv_allocated_len = len(terminal)
    return slots


def materialize_decode_reuse(req, model_runner):
    """Copy + RoPE of the reused versions that moved, all layers at once,
    before the metadata is published."""
    reuse = getattr(req, "context_decode_reuse", None)
    if reuse is None or not len(reuse.copy_indices):
        return
    binding = getattr(model_runner, "context_model_binding", None)
    if binding is None:
        binding = ContextModelBinding(model_runner.model, model_runner.token_to_kv_pool,
                                      model_runner.kv_index_translator, page_size=1)
        model_runner.context_model_binding = binding
    state_slots = req.context_state.slots
    raw = req.context_decode_layout.raw_indices[reuse.copy_indices].astype(np.int64)
    g = _Gather(state_slots.device, state_slots.dtype)
    b = g.request(reuse.source_slots.to(state_slots.dtype), state_slots)
    g.add(b, raw, narrow=True)
    g.add(b, len(reuse.source_slots) + reuse.copy_indices.astype(np.int64), narrow=True)
    _, (src, dst), _ = g.run()
    binding.reposition_existing(src, dst, reuse.position_pairs.to(state_slots.device))
