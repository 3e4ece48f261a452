"""Test-side callers of the akv_amd drop-ins.

In a deployment the reference's own host classes (its decode registry,
layer binding and prefill metadata builder) call the akv_amd entry points
unchanged.  The tests play that caller with these helpers, written for the
tests: they pack the inputs the entry points take and nothing more (no
engine objects, no validation of engine state).
"""

from types import SimpleNamespace

import numpy as np
import torch

from akv_amd import ops, page_table

# ---------------------------------------------------------------------------
# Decode: registry rows and read indices.
#
# Each row the decode-index kernels read is int64
# (raw_ids_ptr, positions_ptr, prompt_len, active, next_pos, row_ptr); a row
# of zeros is an ordinary request read straight from its table row.


class DecodeRows:
    """Registry rows of a batch, with the device arrays they point into."""

    def __init__(self, rows, keep_alive, host):
        self.rows = rows  # int64 [n, 6] on the device, indexed by row id
        self.keep_alive = keep_alive
        self.host = host  # device pointer -> host copy of the pointed-to array

    @classmethod
    def from_layouts(cls, n_rows, entries, device):
        """``entries``: (row_id, layout or None); a layout's final active
        versions (raw index, position) go to the device in one copy."""
        raw_parts, pos_parts, spans = [], [], []
        at = 0
        for _, lay in entries:
            if lay is None:
                spans.append(None)
                continue
            raw = np.flatnonzero(np.asarray(lay.keep_mask)).astype(np.int32)
            raw_parts.append(raw)
            pos_parts.append(np.asarray(lay.positions)[raw].astype(np.int32))
            spans.append((at, len(raw)))
            at += len(raw)
        flat = np.concatenate(raw_parts + pos_parts) if raw_parts else np.zeros(1, np.int32)
        dev = torch.from_numpy(flat).to(device)
        table = np.zeros((n_rows, 6), dtype=np.int64)
        host = {}
        for (row, lay), span in zip(entries, spans):
            if lay is None:
                continue
            start, count = span
            raw_ptr = dev.data_ptr() + 4 * start
            pos_ptr = dev.data_ptr() + 4 * (at + start)
            table[row] = (raw_ptr, pos_ptr, len(lay.positions), count, lay.next_position, 0)
            host[raw_ptr] = flat[start:start + count]
            host[pos_ptr] = flat[at + start:at + start + count]
        return cls(torch.from_numpy(table).to(device), dev, host)


def window_indices(rows, table, row_ids, seq_lens, window, indptr, output, *, mapping=None, multiplier=1,
                   status=None):
    """Sliding-window read indices: visible counts, their offsets, the slots."""
    lengths = torch.empty_like(seq_lens)
    starts = torch.empty_like(seq_lens)
    page_table.context_window_lengths(rows, row_ids, seq_lens, lengths, window, starts=starts)
    indptr = indptr[: len(seq_lens) + 1]
    page_table.build_indptr(lengths, indptr)
    page_table.context_decode_indices(rows, table, row_ids, lengths, indptr, output, starts=starts,
                                      mapping=mapping, multiplier=multiplier, status=status)
    return indptr, lengths, starts


def dense_indices(rows, table, row_ids, seq_lens, output, *, window=None):
    """The page-one dense table form: request b's slots in ``output[b]``."""
    lengths, starts = seq_lens, None
    if window is not None:
        lengths = torch.empty_like(seq_lens)
        starts = torch.empty_like(seq_lens)
        page_table.context_window_lengths(rows, row_ids, seq_lens, lengths, window, starts=starts)
    indptr = torch.empty(len(seq_lens) + 1, dtype=torch.int32, device=seq_lens.device)
    page_table.table_indptr(len(seq_lens), output.stride(0), indptr)
    page_table.context_decode_indices(rows, table, row_ids, lengths, indptr, output.view(-1), starts=starts)
    return lengths


# ---------------------------------------------------------------------------
# Prefill: attention metadata from occurrence windows.


def window_segments(window):
    """Query segments of one occurrence window and the keys each reads
    before its own births.

    A segment's key list ends in the births of its queries, so its prefix
    is the list without its last (query count) entries.
    """
    q_start = np.asarray(window.segment_query_starts, dtype=np.int64)
    q_end = np.asarray(window.segment_query_ends, dtype=np.int64)
    keys = np.asarray(window.segment_key_occurrences, dtype=np.int64)
    key_off = np.asarray(window.segment_key_offsets, dtype=np.int64)
    positions = np.asarray(window.occurrence_positions, dtype=np.int64)
    births = np.asarray(window.birth_occurrences, dtype=np.int64)
    n_query = q_end - q_start
    n_keys = np.diff(key_off)
    n_prefix = n_keys - n_query
    segment_of_key = np.repeat(np.arange(len(n_query)), n_keys)
    rank_in_segment = np.arange(len(keys)) - key_off[:-1][segment_of_key]
    prefix = keys[rank_in_segment < n_prefix[segment_of_key]]
    return SimpleNamespace(
        query_lengths=n_query, prefix_lengths=n_prefix, prefix=prefix,
        query_positions=positions[births[q_start[0]:q_end[-1]]], prefix_positions=positions[prefix],
        occurrences=len(np.asarray(window.occurrence_raw_tokens)))


def plain_segments(prefix_length, query_length):
    """A request without drops: ``prefix_length`` keys, then its queries."""
    keys = np.arange(prefix_length, dtype=np.int64)
    return SimpleNamespace(
        query_lengths=np.array([query_length]), prefix_lengths=np.array([prefix_length]), prefix=keys,
        query_positions=np.arange(prefix_length, prefix_length + query_length, dtype=np.int64),
        prefix_positions=keys.copy(), occurrences=prefix_length + query_length)


def attention_metadata(requests, occurrence_slots):
    """Batch metadata for ``extend_attention_fwd``: the requests' segments in
    order, their prefixes bound to physical slots (one slot per occurrence
    of the batch, request after request)."""
    device = occurrence_slots.device
    q_len = np.concatenate([r.query_lengths for r in requests])
    p_len = np.concatenate([r.prefix_lengths for r in requests])
    base = np.cumsum([0] + [r.occurrences for r in requests])[:-1]
    occurrences = np.concatenate([r.prefix + b for r, b in zip(requests, base)])
    cpu = SimpleNamespace(
        qo_indptr=np.concatenate(([0], np.cumsum(q_len))).astype(np.int64),
        kv_indptr=np.concatenate(([0], np.cumsum(p_len))).astype(np.int64),
        occurrences=occurrences.astype(np.int64),
        query_positions=np.concatenate([r.query_positions for r in requests]),
        kv_positions=np.concatenate([r.prefix_positions for r in requests]))
    dev = {k: torch.from_numpy(np.ascontiguousarray(v)).to(device) for k, v in vars(cpu).items()}
    return SimpleNamespace(
        qo_indptr=dev["qo_indptr"], kv_indptr=dev["kv_indptr"],
        kv_indices=occurrence_slots.index_select(0, dev["occurrences"]),
        query_positions=dev["query_positions"], kv_positions=dev["kv_positions"],
        query_count=int(q_len.sum()), max_query_length=int(q_len.max()), cpu=cpu)


# ---------------------------------------------------------------------------
# Reposition: layers of one model in compatible groups.


def reposition_groups(layers, sources, destinations, pairs):
    """One ``reposition_kv_layers`` launch per group of layers that share a
    K/V geometry, dtype, rotary table and slot translation.

    ``layers``: objects with ``k``, ``v``, ``table``, ``is_neox``,
    ``rotary_dim`` and ``to_slots`` (None, or an int64 device map from the
    caller's slot ids to this layer's pool, 0 where it holds no copy).
    Returns the number of launches.
    """
    groups = {}
    for layer in layers:
        key = (layer.k.dtype, tuple(layer.k.shape[1:]), layer.k.stride(), layer.v.stride(),
               layer.table.data_ptr(), layer.is_neox, layer.rotary_dim,
               None if layer.to_slots is None else layer.to_slots.data_ptr())
        groups.setdefault(key, []).append(layer)
    for members in groups.values():
        first = members[0]
        device = first.k.device
        k_ptrs = torch.tensor([m.k.data_ptr() for m in members], dtype=torch.int64, device=device)
        v_ptrs = torch.tensor([m.v.data_ptr() for m in members], dtype=torch.int64, device=device)
        src, dst = sources, destinations
        if first.to_slots is not None:
            src = first.to_slots[sources.long()].to(torch.int32)
            dst = first.to_slots[destinations.long()].to(torch.int32)
        ops.reposition_kv_layers(k_ptrs, v_ptrs, first.k, first.v, src, dst, pairs, first.table,
                                 is_neox_style=first.is_neox, skip_unmapped=first.to_slots is not None,
                                 rotary_dim=first.rotary_dim)
    return len(groups)


def prefill_forward(meta, q, k_extend, v_extend, output, k_pool, v_pool, **kwargs):
    """One ``extend_attention_fwd`` launch over ``attention_metadata``."""
    from akv_amd import context_attention

    context_attention.extend_attention_fwd(
        q, k_extend, v_extend, output, k_pool, v_pool, meta.qo_indptr, meta.kv_indptr, meta.kv_indices,
        None, True, None, meta.max_query_length,
        context_q_positions=meta.query_positions, context_kv_positions=meta.kv_positions, **kwargs)
    return output
