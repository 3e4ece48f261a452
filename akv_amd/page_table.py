"""Decode metadata over compacted request rows (host side of the HIP kernels).

Mirrors the reference's decode-index path:

* ``context_decode_indices`` / ``context_window_lengths``
  (``akv/system/sglang/kernels/ops/attention/context_page_table.py:7-76``)
  -> ``akv_decode_indices`` / ``akv_window_lengths``;
* ``kv_indptr[1:] = cumsum(seq_lens)`` (``akv/system/sglang.patch:2266-2268``)
  -> ``akv_build_indptr``;
* ``ReqToTokenPool.write`` through side rows (``sglang.patch:4230-4235``)
  -> ``akv_write_row_slots``.

The reference's decode registry (``context_backend.py:666-809``) calls these
with its own int64 rows ``(raw_ids_ptr, positions_ptr, prompt_len, active,
next_pos, row_ptr)``, one per request-table row; a row of zeros is an
ordinary request read straight from its table row.
"""

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


def _status_ptr(status, device):
    if status is None:
        return None
    if status.dtype != torch.int32 or status.numel() < 1 or status.device != device:
        raise ValueError("status must be an int32 device word on the output's device")
    return status.data_ptr()


def context_decode_indices(registry, table, rows, lengths, indptr, output, *, starts=None,
                           mapping=None, multiplier=1, status=None):
    """``out[indptr[b] + i] = T(row[raw])`` over ``len(lengths)`` requests.

    ``status``: the compaction's device status word when the registry rows
    point at its decode layout; the kernel then skips its reads and writes
    on the device when that compaction's outputs are unusable."""
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
            _status_ptr(status, device), current_stream_handle(device),
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


def write_req_to_token_pool(req_to_token, req_pool_indices, prefix_tensors, pre_lens, seq_lens, extend_lens,
                            out_cache_loc, row_pointers=None, *, prefix_dtype=torch.int64):
    """Extend write of request rows: ``write_req_to_token_pool_triton`` with
    ``RowPointers`` (``akv/system/sglang.patch:238-278``).

    For request ``b`` (table row ``r = req_pool_indices[b]``, or the side row
    ``row_pointers[r]`` when given): the first ``pre_lens[b]`` entries come
    from the array at address ``prefix_tensors[b]`` (``prefix_dtype``), the
    next ``seq_lens[b] - pre_lens[b]`` from ``out_cache_loc`` after the
    earlier requests' ``extend_lens``.
    """
    if req_to_token.dtype != torch.int32 or req_to_token.stride(-1) != 1:
        raise ValueError("the request table must be int32 with unit column stride")
    if prefix_tensors.dtype != torch.int64 or (row_pointers is not None and row_pointers.dtype != torch.int64):
        raise ValueError("prefix tensors and row pointers must be int64 addresses")
    if pre_lens.dtype != seq_lens.dtype or extend_lens.dtype != seq_lens.dtype:
        raise ValueError("pre_lens, seq_lens and extend_lens must share one dtype")
    rows_p, rows_t = _idx(req_pool_indices, "req_pool_indices")
    len_t = _idx(seq_lens, "seq_lens")[1]
    loc_p, loc_t = _idx(out_cache_loc, "out_cache_loc")
    prefix_t = _INDEX_DTYPES.get(prefix_dtype)
    if prefix_t is None:
        raise ValueError("prefix_dtype must be int32 or int64")
    device = req_to_token.device
    with _on_device(device):
        rc = _lib.load().akv_write_extend_rows(
            req_to_token.data_ptr(), req_to_token.stride(0), _lib.ptr(row_pointers), rows_p, rows_t,
            prefix_tensors.data_ptr(), prefix_t, pre_lens.data_ptr(), seq_lens.data_ptr(), extend_lens.data_ptr(),
            len_t, loc_p, loc_t, len(req_pool_indices), current_stream_handle(device),
        )
    _lib.check(rc, "akv_write_extend_rows")
