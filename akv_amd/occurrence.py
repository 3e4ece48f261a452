"""Occurrence windows and the final-forward ownership plan (host side).

``compile_occurrence_window`` keeps the signature, fields and messages of
``akv/system/sglang/srt/context_system/occurrence.py:84-265``; the replay runs
in C++ (``akv_window_count`` / ``akv_window_compile``).  The device binding of
a fresh request's whole-prompt forward -- occurrence slots, copy lists,
terminal row and retired slots, ``occurrence.py:341-755`` for
``query_start = 0, query_end = n`` with every slot request-owned -- runs in
``akv_bind_occurrences``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .ops import _on_device, current_stream_handle


@dataclass(frozen=True)
class OccurrenceWindow:
    """Attention/KV plan of one raw query window (``occurrence.py:84-110``).

    ``first_final_occurrence``: occurrences ``[n, first_final)`` are versions
    a segment reads; later ones are terminal versions materialised after the
    last stage.
    """

    occurrence_raw_tokens: torch.Tensor
    occurrence_positions: torch.Tensor
    birth_occurrences: torch.Tensor
    terminal_occurrences: torch.Tensor
    segment_query_starts: torch.Tensor
    segment_query_ends: torch.Tensor
    segment_key_offsets: torch.Tensor
    segment_key_occurrences: torch.Tensor
    first_final_occurrence: int = 0

    @property
    def occurrence_count(self) -> int:
        return len(self.occurrence_raw_tokens)

    @property
    def segment_count(self) -> int:
        return len(self.segment_query_starts)


def _i32p(t):
    return ctypes.c_void_p(t.data_ptr()) if t.numel() else None


def compile_occurrence_window(layout, full_token_visible_until, terminal_positions, *, query_start, query_end,
                             keys_capacity=None):
    """Same ordered plan as the reference, from request-local CPU int32 arrays.

    ``keys_capacity`` (optional) sizes the first replay's key array; the
    default is four keys per token before ``query_end``.
    """
    tensors = (
        layout.birth_positions,
        layout.birth_stages,
        layout.transition_offsets,
        layout.transition_raw_tokens,
        layout.transition_old_positions,
        layout.transition_new_positions,
        full_token_visible_until,
        terminal_positions,
    )
    if any(t.device.type != "cpu" or t.dtype != torch.int32 or t.ndim != 1 for t in tensors):
        raise ValueError("Compact occurrence inputs must be one-dimensional CPU int32 tensors.")
    birth, stages, offsets, changed, old, new, expiry, terminal = (t.contiguous() for t in tensors)
    n = len(birth)
    if n < 1 or len(stages) != n:
        raise ValueError("Compact occurrence birth metadata must cover a nonempty prompt.")
    if len(expiry) != n or len(terminal) != n:
        raise ValueError("Occurrence visibility and terminal positions must cover the prompt.")
    if not 0 <= query_start < query_end <= n:
        raise ValueError("Occurrence query window is outside the raw prompt.")
    if len(offsets) < 1:
        raise ValueError("Occurrence transition offsets require an initial zero.")
    if int(offsets[0]) != 0 or bool((offsets[1:] < offsets[:-1]).any()):
        raise ValueError("Occurrence transition offsets must start at zero and be monotonic.")
    if not int(offsets[-1]) == len(changed) == len(old) == len(new):
        raise ValueError("Occurrence transition offsets do not cover the transition arrays.")
    lib = _lib.load()
    args = (n, _i32p(birth), _i32p(stages), _i32p(offsets), len(offsets) - 1, _i32p(changed), _i32p(old),
            _i32p(new), _i32p(expiry), _i32p(terminal), int(query_start), int(query_end))
    # one replay into arrays sized by the bounds (occurrences <= n + transitions,
    # segments <= queries) and a guess for the keys; a second, exact replay
    # only when the keys outgrow the guess
    caps = np.array([n + len(changed), int(query_end) - int(query_start),
                     keys_capacity if keys_capacity is not None else 4 * int(query_end)], dtype=np.int64)
    counts = np.zeros(4, dtype=np.int64)
    out = _window_arrays(n, caps)
    rc = lib.akv_window_compile_bounded(*args, caps.ctypes.data, counts.ctypes.data, *_window_ptrs(out))
    _lib.check(rc, "akv_window_compile_bounded")
    if (counts[:3] > caps).any():
        out = _window_arrays(n, counts)
        rc = lib.akv_window_compile(*args, counts.ctypes.data, *_window_ptrs(out))
        _lib.check(rc, "akv_window_compile")
    occ, segs, keys, first_final = (int(x) for x in counts)
    out = {k: v[: {"occurrence_raw_tokens": occ, "occurrence_positions": occ, "terminal_occurrences": n,
                   "segment_query_starts": segs, "segment_query_ends": segs, "segment_key_offsets": segs + 1,
                   "segment_key_occurrences": keys}[k]] for k, v in out.items()}
    return OccurrenceWindow(birth_occurrences=torch.arange(n, dtype=torch.int32), first_final_occurrence=first_final,
                            **out)


_WINDOW_FIELDS = ("occurrence_raw_tokens", "occurrence_positions", "terminal_occurrences", "segment_query_starts",
                  "segment_query_ends", "segment_key_offsets", "segment_key_occurrences")


def _window_arrays(n, sizes):
    occ, segs, keys = (int(x) for x in sizes[:3])
    lengths = (occ, occ, n, segs, segs, segs + 1, keys)
    return {k: torch.empty(m, dtype=torch.int32) for k, m in zip(_WINDOW_FIELDS, lengths)}


def _window_ptrs(out):
    # never empty: a window has at least one occurrence, segment and key
    return tuple(ctypes.c_void_p(out[k].data_ptr()) for k in _WINDOW_FIELDS)


# ---------------------------------------------------------------------------
# Device binding of a fresh request's whole-prompt forward.


@dataclass
class FinalForwardInputs:
    """Packed window metadata of a batch (device) plus the host-known counts."""

    bases: torch.Tensor  # int64 [6, B+1]
    occurrence_raw_tokens: torch.Tensor  # int32, request-major
    occurrence_positions: torch.Tensor
    terminal_occurrences: torch.Tensor
    keep: torch.Tensor  # uint8
    n_tokens: tuple
    occurrences: tuple
    extra: tuple  # fresh slots (allocated occurrences) per request
    retired: tuple

    @property
    def n_requests(self):
        return len(self.n_tokens)

    @property
    def max_occurrences(self):
        return max(self.occurrences) if self.occurrences else 0


def final_forward_counts(window, keep):
    """(allocated occurrences, retired birth slots) of a whole-prompt forward."""
    raw = window.occurrence_raw_tokens.numpy()
    pos = window.occurrence_positions.numpy()
    term = window.terminal_occurrences.numpy()
    keep = np.asarray(keep, dtype=bool)
    n = len(term)
    ids = np.arange(len(raw))
    required = (ids < window.first_final_occurrence) | keep[raw]
    alloc = (ids >= n) & required & (pos != pos[raw])
    births_retired = ~(keep & (pos[term] == pos[:n]))
    return int(alloc.sum()), int(births_retired.sum())


def pack_final_forward(windows, keep_masks, device):
    """One host-to-device copy of the windows' binding metadata."""
    if len(windows) != len(keep_masks) or not windows:
        raise ValueError("need one keep mask per window")
    ns, occs, extras, rets, births_ret, finals = [], [], [], [], [], []
    for w, k in zip(windows, keep_masks):
        n = len(w.terminal_occurrences)
        if int(w.segment_query_starts[0]) != 0 or int(w.segment_query_ends[-1]) != n:
            raise ValueError("Occurrence ownership does not cover the planned queries")
        k = np.asarray(k, dtype=bool)
        if len(k) != n:
            raise ValueError("keep mask must cover the prompt")
        extra, br = final_forward_counts(w, k)
        ns.append(n)
        occs.append(w.occurrence_count)
        extras.append(extra)
        births_ret.append(br)
        rets.append(n + extra - int(k.sum()))
        finals.append(w.first_final_occurrence)
    B = len(windows)
    bases = np.zeros((6, B + 1), dtype=np.int64)
    bases[0, 1:] = np.cumsum(occs)
    bases[1, 1:] = np.cumsum(ns)
    bases[2, 1:] = np.cumsum(extras)
    bases[3, 1:] = np.cumsum(rets)
    bases[4, :B] = bases[3, :B] + np.asarray(births_ret)
    bases[4, B] = bases[3, B]
    bases[5, :B] = finals
    total_occ, total_n = int(bases[0, B]), int(bases[1, B])
    words = 2 * bases.size + 2 * total_occ + total_n + (total_n + 3) // 4
    packed = np.zeros(words, dtype=np.int32)
    packed[: 2 * bases.size] = bases.reshape(-1).view(np.int32)
    at = 2 * bases.size
    packed[at : at + total_occ] = np.concatenate([w.occurrence_raw_tokens.numpy() for w in windows])
    packed[at + total_occ : at + 2 * total_occ] = np.concatenate([w.occurrence_positions.numpy() for w in windows])
    at2 = at + 2 * total_occ
    packed[at2 : at2 + total_n] = np.concatenate([w.terminal_occurrences.numpy() for w in windows])
    at3 = at2 + total_n
    packed[at3:].view(np.uint8)[:total_n] = np.concatenate([np.asarray(k, dtype=np.uint8) for k in keep_masks])
    # one staged copy from pageable memory (a fresh pinned buffer per call
    # costs more than the copy of this size)
    dev = torch.from_numpy(packed).to(device, non_blocking=True)
    return FinalForwardInputs(
        bases=dev[: 2 * bases.size].view(torch.int64).view(6, B + 1),
        occurrence_raw_tokens=dev[at : at + total_occ],
        occurrence_positions=dev[at + total_occ : at + 2 * total_occ],
        terminal_occurrences=dev[at2 : at2 + total_n],
        keep=dev[at3:].view(torch.uint8)[:total_n],
        n_tokens=tuple(ns), occurrences=tuple(occs), extra=tuple(extras), retired=tuple(rets),
    )


@dataclass
class FinalForwardOutputs:
    occurrence_slots: torch.Tensor
    copy_src: torch.Tensor
    copy_dst: torch.Tensor
    copy_pairs: torch.Tensor
    retired: torch.Tensor
    workspace: torch.Tensor


def allocate_final_forward_outputs(inputs, device):
    lib = _lib.load()
    i32 = torch.int32
    m = sum(inputs.extra)
    ws = lib.akv_bind_workspace_bytes(inputs.n_requests, inputs.max_occurrences)
    return FinalForwardOutputs(
        occurrence_slots=torch.empty(sum(inputs.occurrences), dtype=i32, device=device),
        copy_src=torch.empty(m, dtype=i32, device=device),
        copy_dst=torch.empty(m, dtype=i32, device=device),
        copy_pairs=torch.empty((m, 2), dtype=i32, device=device),
        retired=torch.empty(sum(inputs.retired), dtype=i32, device=device),
        workspace=torch.empty(max(1, (ws + 3) // 4), dtype=i32, device=device),
    )


def bind_final_forward(inputs, req_to_token, req_rows, birth_slots, fresh_slots, outputs, *, row_pointers=None):
    """Bind slots for every occurrence and write each request's terminal row.

    ``birth_slots``: int32 per raw token (request-major, the extend's write
    slots); ``fresh_slots``: int32, ``inputs.extra[b]`` per request.
    """
    if req_to_token.dtype != torch.int32 or req_to_token.ndim != 2 or req_to_token.stride(1) != 1:
        raise ValueError("req_to_token must be an int32 [rows, width] table with unit column stride")
    if row_pointers is None and req_to_token.shape[1] < max(inputs.n_tokens):
        raise ValueError("req_to_token rows are shorter than the longest request")
    if row_pointers is not None and row_pointers.dtype != torch.int64:
        raise ValueError("row_pointers must be int64 addresses")
    if req_rows.dtype != torch.int64 or req_rows.shape != (inputs.n_requests,):
        raise ValueError("req_rows must be int64 [B]")
    if birth_slots.dtype != torch.int32 or birth_slots.shape != (sum(inputs.n_tokens),):
        raise ValueError("birth_slots must be int32 with one slot per raw token")
    if fresh_slots.dtype != torch.int32 or fresh_slots.shape != (sum(inputs.extra),):
        raise ValueError("Context admission does not cover the selected window")
    lib = _lib.load()
    device = req_to_token.device
    with _on_device(device):
        rc = lib.akv_bind_occurrences(
            inputs.n_requests, inputs.bases.data_ptr(), inputs.max_occurrences,
            inputs.occurrence_raw_tokens.data_ptr(), inputs.occurrence_positions.data_ptr(),
            inputs.terminal_occurrences.data_ptr(), inputs.keep.data_ptr(), birth_slots.data_ptr(),
            _lib.ptr(fresh_slots) if fresh_slots.numel() else None,
            outputs.occurrence_slots.data_ptr(), outputs.copy_src.data_ptr(), outputs.copy_dst.data_ptr(),
            outputs.copy_pairs.data_ptr(), outputs.retired.data_ptr(), req_to_token.data_ptr(),
            req_to_token.stride(0), _lib.ptr(row_pointers), req_rows.data_ptr(), outputs.workspace.data_ptr(),
            outputs.workspace.numel() * 4, current_stream_handle(device),
        )
    _lib.check(rc, "akv_bind_occurrences")
    return outputs
