"""Batched page-table compaction after Drop + Reposition (host side).

The device work runs in ``akv_compact_rows`` (``libakv_amd.so``).  This
module packs the CPU-known per-request metadata (keep mask, birth and final
positions -- all from the compiled layout) into one host-to-device copy, like
the reference's packed transfers (``occurrence.py:721-736``), allocates the
outputs whose sizes the CPU layout already fixes, and launches.

Semantics per request (single-owner final forward, ``occurrence.py:632-767``):

* raw row, in place:  ``keep ? (moved ? fresh : birth) : -1`` (``terminal_slots``);
* retired:            birth slots of dropped or moved tokens, raw order;
* copies:             ``(birth slot, fresh slot, (birth pos, final pos))`` of
                      moved tokens -- exactly the Reposition inputs;
* decode layout:      ``raw_indices = flatnonzero(keep)`` and their positions
                      (``ContextDecodeLayout.from_layout``, ``occurrence.py:47-66``);
* ``kv_indices``:     the compacted row, then ``generated`` raw entries after the
                      prompt (``request_active_slots``, ``context_transfer.py:110-128``),
                      laid out by ``kv_indptr``.
"""

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .ops import _on_device, current_stream_handle


@dataclass
class CompactionInputs:
    """Device copies of the per-token metadata of a batch (request-major)."""

    req_offsets: torch.Tensor  # int64 [B+1]
    keep: torch.Tensor  # uint8 [N]
    birth_positions: torch.Tensor  # int32 [N]
    final_positions: torch.Tensor  # int32 [N]
    n_tokens: tuple
    kept: tuple
    moved: tuple
    max_tokens: int

    @property
    def n_requests(self):
        return len(self.n_tokens)

    @property
    def kept_total(self):
        return sum(self.kept)

    @property
    def moved_total(self):
        return sum(self.moved)

    @property
    def retired_total(self):
        return sum(n - k + m for n, k, m in zip(self.n_tokens, self.kept, self.moved))


def pack_compaction_inputs(layouts, device):
    """One host-to-device copy of every request's keep / birth / final arrays.

    ``layouts``: objects with CPU ``keep_mask``, ``birth_positions`` and
    ``positions`` (a ``ContextLayout``).
    """
    keeps, births, finals, ns, kept, moved = [], [], [], [], [], []
    for layout in layouts:
        keep = np.asarray(layout.keep_mask, dtype=bool)
        birth = np.asarray(layout.birth_positions, dtype=np.int32)
        final = np.asarray(layout.positions, dtype=np.int32)
        keeps.append(keep)
        births.append(birth)
        finals.append(final)
        ns.append(len(keep))
        kept.append(int(keep.sum()))
        moved.append(int((keep & (birth != final)).sum()))
    total = sum(ns)
    offsets = np.zeros(len(ns) + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(ns)
    # int32 words: birth | final | offsets (as 2 words each) | keep (bytes, padded)
    keep_words = (total + 3) // 4
    packed = np.zeros(2 * total + 2 * len(offsets) + keep_words, dtype=np.int32)
    packed[:total] = np.concatenate(births) if total else []
    packed[total : 2 * total] = np.concatenate(finals) if total else []
    packed[2 * total : 2 * total + 2 * len(offsets)] = offsets.view(np.int32)
    keep_bytes = packed[2 * total + 2 * len(offsets) :].view(np.uint8)
    if total:
        keep_bytes[:total] = np.concatenate(keeps).astype(np.uint8)
    # one staged copy from pageable memory (a fresh pinned buffer per call
    # costs more than the copy of this size)
    dev = torch.from_numpy(packed).to(device, non_blocking=True)
    off = 2 * total
    return CompactionInputs(
        req_offsets=dev[off : off + 2 * len(offsets)].view(torch.int64),
        keep=dev[off + 2 * len(offsets) :].view(torch.uint8)[:total],
        birth_positions=dev[:total],
        final_positions=dev[total : 2 * total],
        n_tokens=tuple(ns),
        kept=tuple(kept),
        moved=tuple(moved),
        max_tokens=max(ns) if ns else 0,
    )


@dataclass
class CompactionOutputs:
    retired: torch.Tensor
    copy_src: torch.Tensor
    copy_dst: torch.Tensor
    copy_pairs: torch.Tensor
    raw_indices: torch.Tensor
    active_positions: torch.Tensor
    kv_indices: torch.Tensor | None
    kv_indptr: torch.Tensor | None
    last_page_len: torch.Tensor | None
    counts: torch.Tensor
    status: torch.Tensor
    workspace: torch.Tensor


def allocate_outputs(inputs, device, *, generated_total=None):
    """Outputs of exactly the sizes the CPU layouts fix (no device read-back)."""
    lib = _lib.load()
    i32 = torch.int32
    ws_bytes = lib.akv_compact_workspace_bytes(inputs.n_requests, sum(inputs.n_tokens))
    kv = None
    indptr = None
    if generated_total is not None:
        kv = torch.empty(inputs.kept_total + generated_total, dtype=i32, device=device)
        indptr = torch.empty(inputs.n_requests + 1, dtype=i32, device=device)
    return CompactionOutputs(
        retired=torch.empty(inputs.retired_total, dtype=i32, device=device),
        copy_src=torch.empty(inputs.moved_total, dtype=i32, device=device),
        copy_dst=torch.empty(inputs.moved_total, dtype=i32, device=device),
        copy_pairs=torch.empty((inputs.moved_total, 2), dtype=i32, device=device),
        raw_indices=torch.empty(inputs.kept_total, dtype=i32, device=device),
        active_positions=torch.empty(inputs.kept_total, dtype=i32, device=device),
        kv_indices=kv,
        kv_indptr=indptr,
        last_page_len=None if indptr is None else torch.empty(inputs.n_requests, dtype=i32, device=device),
        counts=torch.empty((inputs.n_requests, 3), dtype=i32, device=device),
        # outputs no compaction has written yet are unusable: a gated consumer
        # launched before the first compaction does nothing
        status=torch.full((1,), _lib.AKV_STATUS_INCOMPLETE, dtype=i32, device=device),
        workspace=torch.zeros(max(8, (ws_bytes + 7) // 8), dtype=torch.int64, device=device),
    )


def compact_rows(inputs, req_to_token, req_rows, fresh_slots, outputs, *, row_pointers=None,
                 generated=None, birth_slots=None, page_size=1):
    """Rewrite each request's raw row to its terminal form and emit the lists.

    ``req_to_token``: int32 ``[pool_rows, width]`` request table (rows hold the
    birth slots on entry).  ``req_rows``: int64 ``[B]`` pool row per request.
    ``fresh_slots``: int32 ``[M]`` fresh slots, request-major raw order of the
    moved tokens.  ``row_pointers``: optional int64 ``[pool_rows]`` side-row
    table (``RowPointers``, ``akv/system/sglang.patch:242-278``).  ``generated``:
    optional int32 ``[B]`` count of generated entries to append per request.
    ``birth_slots``: optional int32 flat birth slots (request-major, like the
    keep mask); when given the raw rows are only written, never read, so the
    call can be repeated on the same inputs.
    """
    if req_to_token.dtype != torch.int32 or req_to_token.ndim != 2 or req_to_token.stride(1) != 1:
        raise ValueError("req_to_token must be an int32 [rows, width] table with unit column stride")
    if req_rows.dtype != torch.int64 or req_rows.shape != (inputs.n_requests,):
        raise ValueError("req_rows must be int64 [B]")
    if fresh_slots.dtype != torch.int32 or fresh_slots.shape != (inputs.moved_total,):
        raise ValueError("fresh_slots must be int32 with one slot per moved token")
    if row_pointers is not None and row_pointers.dtype != torch.int64:
        raise ValueError("row_pointers must be int64 addresses")
    if generated is not None and (generated.dtype != torch.int32 or generated.shape != (inputs.n_requests,)):
        raise ValueError("generated must be int32 [B]")
    if birth_slots is not None and (birth_slots.dtype != torch.int32
                                    or birth_slots.shape != (sum(inputs.n_tokens),)):
        raise ValueError("birth_slots must be int32 with one slot per raw token")
    if generated is not None and outputs.kv_indices is None:
        raise ValueError("generated entries need kv_indices outputs")
    if row_pointers is None and req_to_token.shape[1] < inputs.max_tokens:
        raise ValueError("req_to_token rows are shorter than the longest request")
    lib = _lib.load()
    device = req_to_token.device
    with _on_device(device):
        rc = lib.akv_compact_rows(
            inputs.n_requests,
            inputs.req_offsets.data_ptr(),
            sum(inputs.n_tokens),
            req_to_token.data_ptr(),
            req_to_token.stride(0),
            _lib.ptr(row_pointers),
            req_rows.data_ptr(),
            inputs.keep.data_ptr(),
            inputs.birth_positions.data_ptr(),
            inputs.final_positions.data_ptr(),
            _lib.ptr(birth_slots),
            _lib.ptr(fresh_slots) if inputs.moved_total else None,
            inputs.moved_total,
            outputs.retired.data_ptr(),
            outputs.retired.numel(),
            outputs.copy_src.data_ptr(),
            outputs.copy_dst.data_ptr(),
            outputs.copy_pairs.data_ptr(),
            outputs.raw_indices.data_ptr(),
            outputs.active_positions.data_ptr(),
            outputs.raw_indices.numel(),
            _lib.ptr(generated),
            _lib.ptr(outputs.kv_indices),
            outputs.kv_indices.numel() if outputs.kv_indices is not None else 0,
            _lib.ptr(outputs.kv_indptr),
            _lib.ptr(outputs.last_page_len),
            int(page_size),
            outputs.counts.data_ptr(),
            outputs.workspace.data_ptr(),
            outputs.workspace.numel() * 8,
            outputs.status.data_ptr(),
            current_stream_handle(device),
        )
    _lib.check(rc, "akv_compact_rows")
    return outputs


_STATUS_BITS = (
    (_lib.AKV_STATUS_SIZES, "fresh slot count or an output capacity does not match the batch"),
    (_lib.AKV_STATUS_INCOMPLETE, "an output was not written"),
)


def check_status(outputs):
    """Host-side check of a finished compaction, for tests and diagnostics:
    waits for the device (one 4-byte read) and raises when the status word
    marks the outputs unusable; returns the word (bit
    ``AKV_STATUS_REBUILT`` only says that the one-pass path's finishing
    launch rebuilt some tiles).  The hot path never calls it: consumers read
    the word on the device through their ``status`` argument and skip their
    work when it is set."""
    code = int(outputs.status.item())
    if code & _lib.AKV_STATUS_UNUSABLE:
        why = "; ".join(text for bit, text in _STATUS_BITS if code & bit)
        raise RuntimeError(f"akv_compact_rows status {code}: {why}")
    return code


# ---------------------------------------------------------------------------
# Page-granular compaction with copy-on-write (page_size > 1).


@dataclass
class PagedInputs:
    """Device metadata of a paged batch plus the per-request counts (host)."""

    req_offsets: torch.Tensor  # int64 [B+1]
    keep: torch.Tensor  # uint8 [N]
    birth_positions: torch.Tensor  # int32 [N]
    final_positions: torch.Tensor  # int32 [N]
    bases: torch.Tensor  # int64 [6, B+1]
    page_size: int
    n_tokens: tuple
    kept: tuple
    first_copied_page: tuple
    copies: tuple
    fresh_pages: tuple
    new_pages: tuple
    released_pages: tuple

    @property
    def n_requests(self):
        return len(self.n_tokens)

    @property
    def max_tokens(self):
        return max(self.n_tokens) if self.n_tokens else 0


def _paged_counts(keep, birth, final, page_size):
    n = len(keep)
    kept = int(keep.sum())
    if not np.array_equal(final[keep], np.arange(kept)):
        raise ValueError("paged compaction needs compact final positions (a closing Reposition)")
    dropped = np.flatnonzero(~keep)
    p0 = int(dropped[0]) // page_size if len(dropped) else -(-n // page_size)
    copy_from = p0 * page_size
    # pages below p0 stay in place, unrotated: their tokens must already sit
    # at their final positions
    if not np.array_equal(birth[:copy_from], np.arange(min(n, copy_from))):
        raise ValueError("paged compaction keeps the pages before the first drop in place: their tokens' "
                         "birth positions must equal their ranks")
    copies = max(0, kept - copy_from)
    new_pages = -(-kept // page_size)
    fresh = max(0, new_pages - p0)
    released = max(0, -(-n // page_size) - p0)
    return kept, p0, copy_from, copies, fresh, new_pages, released


def pack_paged_inputs(layouts, page_size, device):
    """One host-to-device copy of keep / birth / final plus the per-request bases.

    Request ``b`` keeps logical pages ``< p0_b`` (``p0`` = page of its first
    dropped token) and moves every kept token of rank ``>= p0_b * P`` into
    fresh pages; all offsets follow from the CPU layout.
    """
    if page_size < 1:
        raise ValueError("page_size must be positive")
    keeps, births, finals, stats = [], [], [], []
    for layout in layouts:
        keep = np.asarray(layout.keep_mask, dtype=bool)
        final = np.asarray(layout.positions, dtype=np.int32)
        birth = np.asarray(layout.birth_positions, dtype=np.int32)
        keeps.append(keep)
        births.append(birth)
        finals.append(final)
        stats.append((len(keep),) + _paged_counts(keep, birth, final, page_size))
    B = len(stats)
    ns = [s[0] for s in stats]
    bases = np.zeros((6, B + 1), dtype=np.int64)
    bases[0, :B] = [s[3] for s in stats]  # copy_from
    for row, col in ((1, 1), (2, 4), (3, 5), (4, 6), (5, 7)):
        bases[row, 1:] = np.cumsum([s[col] for s in stats])
    total = sum(ns)
    offsets = np.zeros(B + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(ns)
    keep_words = (total + 3) // 4
    words = 2 * total + 2 * (B + 1) + 2 * bases.size + keep_words
    packed = np.zeros(words, dtype=np.int32)
    at = 0
    for arr in (np.concatenate(births) if total else np.zeros(0, np.int32),
                np.concatenate(finals) if total else np.zeros(0, np.int32)):
        packed[at : at + total] = arr
        at += total
    packed[at : at + 2 * (B + 1)] = offsets.view(np.int32)
    at_off = at
    at += 2 * (B + 1)
    packed[at : at + 2 * bases.size] = bases.reshape(-1).view(np.int32)
    at_bases = at
    at += 2 * bases.size
    if total:
        packed[at:].view(np.uint8)[:total] = np.concatenate(keeps).astype(np.uint8)
    dev = torch.from_numpy(packed).to(device, non_blocking=True)
    return PagedInputs(
        req_offsets=dev[at_off : at_off + 2 * (B + 1)].view(torch.int64),
        keep=dev[at:].view(torch.uint8)[:total],
        birth_positions=dev[:total],
        final_positions=dev[total : 2 * total],
        bases=dev[at_bases : at_bases + 2 * bases.size].view(torch.int64).view(6, B + 1),
        page_size=page_size,
        n_tokens=tuple(ns),
        kept=tuple(s[1] for s in stats),
        first_copied_page=tuple(s[2] for s in stats),
        copies=tuple(s[4] for s in stats),
        fresh_pages=tuple(s[5] for s in stats),
        new_pages=tuple(s[6] for s in stats),
        released_pages=tuple(s[7] for s in stats),
    )


@dataclass
class PagedOutputs:
    copy_src: torch.Tensor
    copy_dst: torch.Tensor
    copy_pairs: torch.Tensor
    released_pages: torch.Tensor
    page_table: torch.Tensor
    raw_indices: torch.Tensor
    active_positions: torch.Tensor


def allocate_paged_outputs(inputs, device):
    i32 = torch.int32
    copies = sum(inputs.copies)
    kept = sum(inputs.kept)
    return PagedOutputs(
        copy_src=torch.empty(copies, dtype=i32, device=device),
        copy_dst=torch.empty(copies, dtype=i32, device=device),
        copy_pairs=torch.empty((copies, 2), dtype=i32, device=device),
        released_pages=torch.empty(sum(inputs.released_pages), dtype=i32, device=device),
        page_table=torch.empty(sum(inputs.new_pages), dtype=i32, device=device),
        raw_indices=torch.empty(kept, dtype=i32, device=device),
        active_positions=torch.empty(kept, dtype=i32, device=device),
    )


def compact_pages(inputs, req_to_token, req_rows, fresh_pages, outputs, *, row_pointers=None, birth_slots=None):
    """Rewrite each request's raw row page-dense; emit copies, released pages and page tables.

    ``fresh_pages``: int32 page ids, request-major, ``inputs.fresh_pages[b]``
    per request (the allocator's pages for the copied logical pages).
    """
    if req_to_token.dtype != torch.int32 or req_to_token.ndim != 2 or req_to_token.stride(1) != 1:
        raise ValueError("req_to_token must be an int32 [rows, width] table with unit column stride")
    if req_rows.dtype != torch.int64 or req_rows.shape != (inputs.n_requests,):
        raise ValueError("req_rows must be int64 [B]")
    if fresh_pages.dtype != torch.int32 or fresh_pages.shape != (sum(inputs.fresh_pages),):
        raise ValueError("fresh_pages must be int32 with one page per copied logical page")
    if birth_slots is not None and (birth_slots.dtype != torch.int32 or birth_slots.shape != (sum(inputs.n_tokens),)):
        raise ValueError("birth_slots must be int32 with one slot per raw token")
    if row_pointers is not None and row_pointers.dtype != torch.int64:
        raise ValueError("row_pointers must be int64 addresses")
    if row_pointers is None and req_to_token.shape[1] < inputs.max_tokens:
        raise ValueError("req_to_token rows are shorter than the longest request")
    sizes = dict(copy_src=(sum(inputs.copies),), copy_dst=(sum(inputs.copies),), copy_pairs=(sum(inputs.copies), 2),
                 released_pages=(sum(inputs.released_pages),), page_table=(sum(inputs.new_pages),),
                 raw_indices=(sum(inputs.kept),), active_positions=(sum(inputs.kept),))
    for name, shape in sizes.items():
        t = getattr(outputs, name)
        if t.dtype != torch.int32 or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"outputs.{name} must be a contiguous int32 tensor of shape {shape}")
    lib = _lib.load()
    device = req_to_token.device
    # an empty list (a batch with nothing copied or released) gets a valid
    # one-element stand-in: the kernel's writes to it are bounded by a zero total
    spare = torch.empty(2, dtype=torch.int32, device=device)

    def out(name):
        t = getattr(outputs, name)
        return t.data_ptr() if t.numel() else spare.data_ptr()

    with _on_device(device):
        rc = lib.akv_compact_pages(
            inputs.n_requests, inputs.req_offsets.data_ptr(), inputs.max_tokens, inputs.page_size,
            req_to_token.data_ptr(), req_to_token.stride(0), _lib.ptr(row_pointers), req_rows.data_ptr(),
            inputs.keep.data_ptr(), inputs.birth_positions.data_ptr(), inputs.final_positions.data_ptr(),
            _lib.ptr(birth_slots), inputs.bases.data_ptr(), _lib.ptr(fresh_pages) if fresh_pages.numel() else None,
            out("copy_src"), out("copy_dst"), out("copy_pairs"), out("released_pages"), out("page_table"),
            out("raw_indices"), out("active_positions"), current_stream_handle(device),
        )
    _lib.check(rc, "akv_compact_pages")
    return outputs
