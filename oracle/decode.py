"""CPU restatement of the decode-metadata kernels over compacted rows.

Restates, as plain Python loops over numpy arrays:

* ``context_decode_indices``
  (``akv/system/sglang/kernels/ops/attention/context_page_table.py:34-76``),
* ``context_window_lengths`` (``:7-31``),
* ``write_row_slots`` (``akv/system/sglang/kernels/ops/memory/context_rows.py:7-15``),
* ``kv_indptr[1:] = cumsum(seq_lens)`` (``akv/system/sglang.patch:2266-2268``)
  and the page-one ``fill_table`` indptr
  (``akv/system/sglang/srt/layers/attention/context_backend.py:785-795``).

Device pointers stored in the int64 registry rows are modelled by a
``memory`` dict that maps a nonzero handle to a numpy int32 array.

Pinned by (``tests/test_oracle_decode.py``): the compacted-row identity --
for a registry row built from a layout, the indices equal
``terminal_row[raw_indices] ++ row[prompt:prompt+generated]`` (the
``request_active_slots`` form, ``context_transfer.py:110-128``) -- the window
lengths against a direct count of positions with ``q_pos - k_pos <= W``, and
``numpy.cumsum`` for the indptr.
"""

import numpy as np


def decode_indices(registry, table, rows, lengths, indptr, output, *, memory,
                   starts=None, mapping=None, multiplier=1):
    """Fill ``output`` in place, one request at a time."""
    for b in range(len(rows)):
        row = int(rows[b])
        length = int(lengths[b])
        offset = int(indptr[b])
        start = 0 if starts is None else int(starts[b])
        pointer, _, prompt, active, _, row_pointer = (int(x) for x in registry[row])
        raw_row = table[row] if row_pointer == 0 else memory[row_pointer]
        raw_ids = memory.get(pointer) if pointer != 0 else None
        active = np.int32(active).item()
        prompt = np.int32(prompt).item()
        for i in range(length):
            logical = start + i
            raw = logical
            if pointer != 0:
                raw = int(raw_ids[logical]) if logical < active else prompt + logical - active
            slot = int(raw_row[raw])
            if mapping is not None:
                slot = int(mapping[slot]) * multiplier
            output[offset + i] = slot


def window_lengths(registry, rows, lengths, window, *, memory):
    """Visible key count per request for a sliding window of ``window``."""
    out = np.zeros(len(rows), dtype=np.int64)
    for b in range(len(rows)):
        row = int(rows[b])
        length = int(lengths[b])
        pointer, positions_ptr, _, active, next_pos, _ = (int(x) for x in registry[row])
        result = min(length, window)
        if pointer != 0:
            positions = memory[positions_ptr]
            active = np.int32(active).item()
            next_pos = np.int32(next_pos).item()
            generated = length - active
            lower = next_pos + generated - 1 - window
            lo, hi = 0, active
            while lo < hi:
                mid = (lo + hi) // 2
                if int(positions[mid]) < lower:
                    lo = mid + 1
                else:
                    hi = mid
            result = active - lo + generated - max(0, lower - next_pos)
        out[b] = result
    return out


def write_row_slots(pointers, rows, columns, values, *, memory):
    for r, c, v in zip(rows, columns, values):
        memory[int(pointers[int(r)])][int(c)] = v


def kv_indptr(lengths):
    out = np.zeros(len(lengths) + 1, dtype=np.int64)
    out[1:] = np.cumsum(np.asarray(lengths, dtype=np.int64))
    return out


def last_page_lengths(lengths, page_size):
    lengths = np.asarray(lengths, dtype=np.int64)
    return np.where(lengths > 0, (lengths - 1) % page_size + 1, 0)
