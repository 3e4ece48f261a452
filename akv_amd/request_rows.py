"""Per-request token rows and their overflow side rows.

Mirror of ``akv/system/sglang/srt/context_system/request_storage.py:240-309``
(``request_row``, ``prepare_request_row``, ``release_request_row``,
``row_pointers``, ``write_request_slots``).  A Context request whose raw
length (prompt + generation budget) exceeds the pool's row width gets a
side row of its own; ``_context_row_pointers`` keeps one device address per
request row, so kernels that take row pointers (``akv_compact_rows``,
``akv_bind_occurrences``, ``akv_write_row_slots``) reach side rows and pool
rows alike.  Batched scatters into rows go through ``akv_write_row_slots``.
"""

from __future__ import annotations

import torch

from .page_table import write_row_slots


def request_row(pool, index):
    """The request's token row, or its side row when it overflowed."""
    rows = getattr(pool, "_context_rows", None)
    if rows and index in rows:
        return rows[index]
    return pool.req_to_token[index]


def prepare_request_row(pool, req):
    """Give a Context request a side row when its raw length can outgrow
    the pool row (the allocation of a discarded overlap step included)."""
    if getattr(req, "context_program", None) is None:
        return
    capacity = len(req.origin_input_ids) + req.sampling_params.max_new_tokens + 4
    if capacity <= pool.req_to_token.shape[1]:
        return
    rows = getattr(pool, "_context_rows", None)
    if rows is None:
        rows = pool._context_rows = {}
    index = req.kv.req_pool_idx
    if index in rows:
        if len(rows[index]) < capacity:
            raise RuntimeError("Context raw row cannot grow while a request is live")
        return
    row = torch.full((capacity,), -1, dtype=torch.int32, device=pool.device)
    rows[index] = row
    if getattr(pool, "_context_row_pointers", None) is None:
        table = pool.req_to_token
        pool._context_row_pointers = (
            torch.arange(table.shape[0], dtype=torch.int64, device=pool.device) * table.stride(0)
            * table.element_size() + table.data_ptr()
        )
    pool._context_row_pointers[index] = row.data_ptr()


def release_request_row(pool, index):
    rows = getattr(pool, "_context_rows", None)
    if rows and index in rows:
        del rows[index]
        pool._context_row_pointers[index] = pool.req_to_token[index].data_ptr()


def row_pointers(pool):
    """Device row addresses when any side row exists, else None."""
    return pool._context_row_pointers if getattr(pool, "_context_rows", None) else None


def write_request_slots(pool, indices, values):
    """``req_to_token[indices] = values`` that also reaches side rows:
    ``indices`` is ``(row, columns)`` with an int row or a tensor of rows."""
    rows = getattr(pool, "_context_rows", None)
    if not rows:
        pool.req_to_token[indices] = values
        return
    row, columns = indices
    if isinstance(row, int):
        request_row(pool, row)[columns] = values
    elif pool.req_to_token.is_cuda:
        write_row_slots(pool._context_row_pointers, row, columns, values)
    else:
        for index, column, value in zip(row.tolist(), columns.tolist(), values):
            request_row(pool, index)[column] = value
