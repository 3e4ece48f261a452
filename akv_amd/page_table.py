"""Decode metadata over compacted request rows (host side of the HIP kernels).

Mirrors the reference's decode-index path:

* ``context_decode_indices`` / ``context_window_lengths``
  (``akv/system/sglang/kernels/ops/attention/context_page_table.py:7-76``)
  -> ``akv_decode_indices`` / ``akv_window_lengths``;
* ``kv_indptr[1:] = cumsum(seq_lens)`` (``akv/system/sglang.patch:2266-2268``)
  -> ``akv_build_indptr``;
* ``ContextDecodeLayout`` (``occurrence.py:36-81``) and
  ``ContextDecodeRegistry`` (``context_backend.py:666-809``) with the same
  ``bind_batch`` / ``fill`` / ``fill_table`` / ``fill_window`` interface.
"""

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .ops import _on_device, current_stream_handle

_INDEX_DTYPES = {torch.int32: _lib.AKV_I32, torch.int64: _lib.AKV_I64}


def _idx(t, name):
    if t is None:
        return None, _lib.AKV_I32
    code = _INDEX_DTYPES.get(t.dtype)
    if code is None or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32/int64 tensor")
    return t.data_ptr(), code


def context_decode_indices(registry, table, rows, lengths, indptr, output, *, starts=None,
                           mapping=None, multiplier=1):
    """``out[indptr[b] + i] = T(row[raw])`` over ``len(lengths)`` requests."""
    if registry.dtype != torch.int64 or registry.ndim != 2 or registry.shape[1] != 6:
        raise ValueError("registry must be int64 [rows, 6]")
    if table.dtype != torch.int32 or table.stride(-1) != 1:
        raise ValueError("the request table must be int32 with unit column stride")
    rows_p, rows_t = _idx(rows, "rows")
    len_p, len_t = _idx(lengths, "lengths")
    ind_p, ind_t = _idx(indptr, "indptr")
    out_p, out_t = _idx(output, "output")
    st_p, st_t = _idx(starts, "starts")
    map_p, map_t = _idx(mapping, "mapping")
    device = output.device
    with _on_device(device):
        rc = _lib.load().akv_decode_indices(
            registry.data_ptr(), table.data_ptr(), table.stride(0), rows_p, rows_t, len_p, len_t,
            ind_p, ind_t, out_p, out_t, st_p, st_t, map_p, map_t, int(multiplier), len(lengths),
            current_stream_handle(device),
        )
    _lib.check(rc, "akv_decode_indices")


def context_window_lengths(registry, rows, lengths, output, window, *, starts=None):
    """Visible key counts for an inclusive ``window``; optionally ``starts = lengths - output``."""
    rows_p, rows_t = _idx(rows, "rows")
    len_p, len_t = _idx(lengths, "lengths")
    out_p, out_t = _idx(output, "output")
    if starts is not None and starts.dtype != lengths.dtype:
        raise ValueError("starts must have the dtype of lengths")
    device = output.device
    with _on_device(device):
        rc = _lib.load().akv_window_lengths(
            registry.data_ptr(), rows_p, rows_t, len_p, len_t, out_p, out_t, _lib.ptr(starts),
            int(window), len(lengths), current_stream_handle(device),
        )
    _lib.check(rc, "akv_window_lengths")


def build_indptr(lengths, indptr, *, last_page_len=None, page_size=1):
    """``indptr[0] = 0; indptr[1:] = cumsum(lengths)`` (+ last-page lengths)."""
    len_p, len_t = _idx(lengths, "lengths")
    ind_p, ind_t = _idx(indptr, "indptr")
    if last_page_len is not None and last_page_len.dtype != torch.int32:
        raise ValueError("last_page_len must be int32")
    device = indptr.device
    with _on_device(device):
        rc = _lib.load().akv_build_indptr(
            len_p, len_t, len(lengths), ind_p, ind_t, _lib.ptr(last_page_len), int(page_size), 1,
            current_stream_handle(device),
        )
    _lib.check(rc, "akv_build_indptr")


def table_indptr(batch, stride, indptr):
    """Page-table form ``indptr[b] = b * stride`` for ``b`` in ``[0, batch]``."""
    ind_p, ind_t = _idx(indptr, "indptr")
    if stride == 1:
        # a scale of 1 would select the cumulative-sum form
        raise ValueError("table_indptr needs a row stride other than 1")
    device = indptr.device
    with _on_device(device):
        rc = _lib.load().akv_build_indptr(
            None, _lib.AKV_I32, batch, ind_p, ind_t, None, 1, int(stride), current_stream_handle(device)
        )
    _lib.check(rc, "akv_build_indptr")


def write_row_slots(pointers, rows, columns, values):
    """``((int32*)pointers[rows[i]])[columns[i]] = values[i]`` (side-row scatter)."""
    if pointers.dtype != torch.int64:
        raise ValueError("row pointers must be int64 addresses")
    rows_p, rows_t = _idx(rows, "rows")
    col_p, col_t = _idx(columns, "columns")
    val_p, val_t = _idx(values, "values")
    device = pointers.device
    with _on_device(device):
        rc = _lib.load().akv_write_row_slots(
            pointers.data_ptr(), rows_p, rows_t, col_p, col_t, val_p, val_t, rows.numel(),
            current_stream_handle(device),
        )
    _lib.check(rc, "akv_write_row_slots")


@dataclass(frozen=True)
class ContextDecodeLayout:
    """Immutable final prompt view; generated KV stays in the native raw row.

    Mirrors ``ContextDecodeLayout`` (``occurrence.py:36-81``).
    """

    raw_indices: np.ndarray
    positions: np.ndarray
    device_indices: torch.Tensor
    device_positions: torch.Tensor
    prompt_length: int
    next_position: int

    @classmethod
    def from_layout(cls, layout, device):
        raw = np.flatnonzero(np.asarray(layout.keep_mask)).astype(np.int32)
        positions = np.asarray(layout.positions)[raw].copy()
        if np.any(np.diff(positions.astype(np.int64)) <= 0):
            raise ValueError("Active decode positions must be strictly increasing")
        packed = torch.from_numpy(np.concatenate((raw, positions.astype(np.int32)))).to(
            device=device, non_blocking=True
        )
        if packed.numel() == 0:
            packed = torch.zeros(1, dtype=torch.int32, device=device)
        return cls(
            raw,
            positions,
            packed[: len(raw)] if len(raw) else packed,
            packed[len(raw):] if len(raw) else packed,
            len(layout.positions),
            layout.next_position,
        )

    @classmethod
    def from_device(cls, raw_indices, positions, device_indices, device_positions, prompt_length,
                    next_position):
        """Bind a layout whose device arrays were produced by ``compact_rows``."""
        return cls(raw_indices, positions, device_indices, device_positions, prompt_length,
                   next_position)

    def swa_raw_floor(self, computed_raw: int, window: int) -> int:
        if computed_raw < self.prompt_length:
            return 0
        generated = computed_raw - self.prompt_length
        lower = self.next_position + generated - 1 - window
        index = int(np.searchsorted(self.positions, lower))
        if index < len(self.raw_indices):
            return int(self.raw_indices[index])
        return self.prompt_length + max(0, lower - self.next_position)


class ContextDecodeRegistry:
    """Capture-stable request-slot registry (``context_backend.py:666-809``).

    ``translator`` needs ``page_size``, ``defer_read_translate``,
    ``req_to_token`` and ``is_translating`` (plus ``_full_v2p_table`` /
    ``_swa_v2p_table`` and their page multipliers when translating);
    ``pool`` may expose ``full_to_swa_index_mapping``; ``request_pool`` may
    hold side rows (``_context_rows``).  Only read indices are compacted; no
    historical KV is copied.
    """

    def __init__(self, translator, pool, request_pool=None):
        if translator.page_size != 1 or translator.defer_read_translate:
            raise ValueError("Context decode requires page_size=1 without DCP")
        self.translator = translator
        self.pool = pool
        self.request_pool = request_pool
        self.rows = torch.zeros(
            (translator.req_to_token.shape[0], 6),
            dtype=torch.int64,
            device=translator.req_to_token.device,
        )
        self.batch_layouts = []

    def bind_batch(self, reqs, raw_lengths, row_ids):
        entries, lengths, positions, refs = [], [], [], []
        self.batch_layouts = []
        for req, raw_length in zip(reqs, raw_lengths):
            raw_length = int(raw_length)
            if req.context_program is None:
                entries.append((0, 0, 0, 0, 0, 0))
                lengths.append(raw_length)
                positions.append(raw_length - 1)
                self.batch_layouts.append((None, raw_length))
                continue
            layout = req.context_decode_layout
            if layout is None:
                layout = ContextDecodeLayout.from_layout(req.context_program.layout, row_ids.device)
                req.context_decode_layout = layout
            generated = raw_length - layout.prompt_length
            if generated < 1:
                raise ValueError("Context decode requires a computed output query")
            count = len(layout.raw_indices)
            row_pointer = 0
            if self.request_pool is not None:
                rows = getattr(self.request_pool, "_context_rows", None)
                index = req.kv.req_pool_idx
                raw_row = rows[index] if rows and index in rows else self.request_pool.req_to_token[index]
                row_pointer = raw_row.data_ptr()
                if raw_row.is_cuda:
                    raw_row.record_stream(torch.cuda.current_stream(raw_row.device))
                refs.append(raw_row)
            entries.append(
                (
                    layout.device_indices.data_ptr(),
                    layout.device_positions.data_ptr(),
                    layout.prompt_length,
                    count,
                    layout.next_position,
                    row_pointer,
                )
            )
            lengths.append(count + generated)
            positions.append(layout.next_position + generated - 1)
            refs.append(layout)
            self.batch_layouts.append((layout, generated))
        packed = torch.tensor(
            [(*entry, n, p) for entry, n, p in zip(entries, lengths, positions)],
            dtype=torch.int64,
        ).to(row_ids.device, non_blocking=True)
        self.rows[row_ids] = packed[:, :6]
        return (
            torch.tensor(lengths, dtype=torch.int64),
            packed[:, 6].to(torch.int32),
            packed[:, 7],
            tuple(refs),
        )

    def window_lengths_cpu(self, window, batch_size):
        lengths = []
        for layout, generated in self.batch_layouts:
            if layout is None:
                lengths.append(min(generated, window + 1))
            else:
                lower = layout.next_position + generated - 1 - window
                start = np.searchsorted(layout.positions, lower)
                lengths.append(len(layout.positions) - start + min(generated, window + 1))
        return torch.tensor(lengths + [1] * (batch_size - len(lengths)), dtype=torch.int64)

    def _mapping(self, swa):
        translator = self.translator
        mapping, multiplier = None, 1
        if getattr(translator, "is_translating", False):
            mapping = translator._swa_v2p_table if swa else translator._full_v2p_table
            multiplier = (
                translator._swa_page_multiplier if swa else translator._full_page_multiplier
            )
        elif swa:
            mapping = getattr(self.pool, "full_to_swa_index_mapping", None)
        return mapping, multiplier

    def fill(self, row_ids, lengths, indptr, output, *, starts=None, swa=False):
        mapping, multiplier = self._mapping(swa)
        context_decode_indices(
            self.rows,
            self.translator.req_to_token,
            row_ids,
            lengths,
            indptr,
            output,
            starts=starts,
            mapping=mapping,
            multiplier=multiplier,
        )

    def fill_table(self, row_ids, seq_lens, output, *, window=None):
        """Fill an existing page-one decode table without raw-row copies."""
        lengths, starts = seq_lens, None
        if window is not None:
            lengths = torch.empty_like(seq_lens)
            starts = torch.empty_like(seq_lens)
            context_window_lengths(self.rows, row_ids, seq_lens, lengths, window, starts=starts)
        indptr = torch.empty(len(seq_lens) + 1, dtype=torch.int32, device=seq_lens.device)
        stride = output.stride(0)
        if stride == 1:
            indptr.copy_(torch.arange(len(seq_lens) + 1, dtype=torch.int32))
        else:
            table_indptr(len(seq_lens), stride, indptr)
        self.fill(row_ids, lengths, indptr, output.view(-1), starts=starts, swa=window is not None)
        return lengths

    def fill_window(self, row_ids, seq_lens, indptr, window, output):
        bs = len(seq_lens)
        lengths = torch.empty_like(seq_lens)
        starts = torch.empty_like(seq_lens)
        context_window_lengths(self.rows, row_ids, seq_lens, lengths, window, starts=starts)
        indptr = indptr[: bs + 1]
        build_indptr(lengths, indptr)
        self.fill(row_ids, lengths, indptr, output, starts=starts, swa=True)
        return indptr, output, lengths, starts
