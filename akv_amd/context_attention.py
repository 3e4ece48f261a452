"""Prefill context attention over occurrence metadata (host side).

Mirrors ``ContextSequence`` / ``ContextAttentionPlan`` /
``ContextAttentionMetadata`` of
``akv/system/sglang/srt/layers/attention/context_backend.py:24-251`` (same
fields, packing, validation and messages) and the extend-attention entry
with context positions (``akv/system/sglang.patch:106-237``).  The device
work is ``akv_context_attention`` in ``libakv_amd.so``; there is no other
path.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .ops import _on_device, current_stream_handle


def _np(x):
    return x.numpy() if isinstance(x, torch.Tensor) else np.asarray(x)


@dataclass(frozen=True)
class ContextSequence:
    """One request's query segments and their visible prefixes (``CB:24-89``)."""

    occurrence_count: int
    query_lengths: tuple
    prefix_offsets: np.ndarray
    prefix_occurrences: np.ndarray
    query_positions: np.ndarray
    prefix_positions: np.ndarray

    @classmethod
    def from_window(cls, window) -> ContextSequence:
        """Convert one validated occurrence window, keeping query order.

        ``window`` carries ``segment_query_starts/ends``,
        ``occurrence_raw_tokens``, ``occurrence_positions``,
        ``birth_occurrences``, ``segment_key_occurrences`` and
        ``segment_key_offsets`` (``OccurrenceWindow``, ``CS/occurrence.py:84-111``).
        """
        starts = _np(window.segment_query_starts)
        ends = _np(window.segment_query_ends)
        if len(starts) == 0 or np.any(ends <= starts):
            raise ValueError("Context attention needs nonempty query segments")
        if not np.array_equal(ends[:-1], starts[1:]):
            raise ValueError("Context attention query segments must be contiguous")
        raw = _np(window.occurrence_raw_tokens)
        positions = _np(window.occurrence_positions)
        birth = _np(window.birth_occurrences)
        keys = _np(window.segment_key_occurrences)
        key_offsets = _np(window.segment_key_offsets)
        prefixes, offsets = [], [0]
        for start, end, a, b in zip(starts, ends, key_offsets[:-1], key_offsets[1:]):
            selected = keys[a:b]
            count = int(end - start)
            if len(selected) < count or not np.array_equal(selected[-count:], birth[start:end]):
                raise ValueError("Context segment must end in its ordered birth KV")
            prefix = selected[:-count]
            if np.any(raw[prefix] >= start):
                raise ValueError("Context prefix cannot read an uncomputed query")
            prefixes.append(prefix)
            offsets.append(offsets[-1] + len(prefix))
        prefix = np.concatenate(prefixes).astype(np.int64, copy=False)
        return cls(
            len(raw),
            tuple(int(n) for n in ends - starts),
            np.asarray(offsets, dtype=np.int64),
            prefix,
            positions[birth[starts[0] : ends[-1]]].astype(np.int64),
            positions[prefix].astype(np.int64),
        )

    @classmethod
    def ordinary(cls, prefix_length: int, query_length: int) -> ContextSequence:
        """An ordinary request: ordered prefix slots, then its query write slots."""
        if prefix_length < 0 or query_length < 1:
            raise ValueError("Invalid ordinary prefix/query lengths")
        prefix = np.arange(prefix_length, dtype=np.int64)
        return cls(
            prefix_length + query_length,
            (query_length,),
            np.asarray([0, prefix_length], dtype=np.int64),
            prefix,
            np.arange(prefix_length, prefix_length + query_length, dtype=np.int64),
            prefix,
        )


@dataclass(frozen=True)
class ContextAttentionPlan:
    """One packed int64 transfer of all segment metadata (``CB:91-165``)."""

    packed: torch.Tensor
    field_ranges: tuple
    query_lengths: tuple
    occurrence_count: int

    @classmethod
    def merge(cls, sequences: Sequence[ContextSequence]) -> ContextAttentionPlan:
        if not sequences:
            raise ValueError("Context attention batch cannot be empty")
        q_lengths, kv_lengths, occurrences, q_pos, kv_pos = [], [], [], [], []
        base = 0
        for seq in sequences:
            q_lengths.extend(seq.query_lengths)
            kv_lengths.append(np.diff(seq.prefix_offsets))
            occurrences.append(seq.prefix_occurrences + base)
            q_pos.append(seq.query_positions)
            kv_pos.append(seq.prefix_positions)
            base += seq.occurrence_count
        fields = (
            np.r_[0, np.cumsum(q_lengths, dtype=np.int64)],
            np.r_[0, np.cumsum(np.concatenate(kv_lengths), dtype=np.int64)],
            np.concatenate(occurrences).astype(np.int64),
            np.concatenate(q_pos).astype(np.int64),
            np.concatenate(kv_pos).astype(np.int64),
        )
        # fields start on 16-byte boundaries; the ranges exclude the padding
        offsets = np.r_[0, np.cumsum([(len(f) + 1) // 2 * 2 for f in fields])]
        packed = np.zeros(int(offsets[-1]), dtype=np.int64)
        ranges = tuple((int(s), int(s) + len(f)) for s, f in zip(offsets, fields))
        for f, (s, e) in zip(fields, ranges):
            packed[s:e] = f
        return cls(torch.from_numpy(packed), ranges, tuple(q_lengths), base)

    def bind(self, occurrence_slots: torch.Tensor) -> ContextAttentionMetadata:
        """Bind physical slots (one per batch occurrence) to the prefixes."""
        if (
            occurrence_slots.ndim != 1
            or occurrence_slots.numel() != self.occurrence_count
            or occurrence_slots.dtype not in (torch.int32, torch.int64)
        ):
            raise ValueError("Physical slot binding must cover all batch occurrences")
        # one staged copy from pageable memory (a fresh pinned buffer per call
        # costs more than the copy of this size)
        packed = self.packed.to(device=occurrence_slots.device, non_blocking=True)
        qo, kv, occurrences, q_positions, kv_positions = [packed[a:b] for a, b in self.field_ranges]
        return ContextAttentionMetadata(
            qo,
            kv,
            occurrence_slots.index_select(0, occurrences),
            q_positions,
            kv_positions,
            self.query_lengths,
            sum(self.query_lengths),
            max(self.query_lengths),
            tuple(self.packed[a:b].numpy() for a, b in self.field_ranges),
        )


@dataclass(frozen=True)
class ContextAttentionMetadata:
    qo_indptr: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    query_positions: torch.Tensor
    kv_positions: torch.Tensor
    query_lengths: tuple
    query_count: int
    max_query_length: int
    cpu_fields: tuple = ()
    native_plans: dict = field(default_factory=dict, compare=False, repr=False)

    def forward(self, kernel, q, k, v, output, k_pool, v_pool, **kwargs):
        """One extend launch, after this layer's KV writes and copy-on-write."""
        if kwargs.get("page_size", 1) != 1:
            raise ValueError("Context attention requires page_size=1")
        if self.query_count != q.shape[0]:
            raise ValueError("Context query metadata does not cover model output")
        kernel(
            q, k, v, output, k_pool, v_pool,
            self.qo_indptr, self.kv_indptr, self.kv_indices,
            None, True, None, self.max_query_length, 1.0, 1.0,
            context_q_positions=self.query_positions,
            context_kv_positions=self.kv_positions,
            extend_seq_lens_cpu=self.query_lengths,
            **kwargs,
        )
        return output


_INDEX = {torch.int32: _lib.AKV_I32, torch.int64: _lib.AKV_I64}


def extend_attention_fwd(q_extend, k_extend, v_extend, o_extend, k_buffer, v_buffer, qo_indptr, kv_indptr,
                         kv_indices, custom_mask, is_causal, mask_indptr, max_len_extend, k_scale=1.0,
                         v_scale=1.0, sm_scale=None, logit_cap=0.0, skip_prefix_custom_mask=True,
                         sliding_window_size=-1, sinks=None, window_kv_offsets=None, xai_temperature_len=-1,
                         extend_seq_lens_cpu=None, context_q_positions=None, context_kv_positions=None,
                         page_size=1):
    """Extend (prefill) attention with context positions, on the HIP kernel.

    Argument order and meaning of the extend attention the context backend
    calls (``akv/system/sglang.patch:893-1157``): ``q_extend`` ``[Nq, Hq, D]``,
    ``k_extend``/``v_extend`` ``[Nq, Hkv, D]`` (this forward's K/V),
    ``k_buffer``/``v_buffer`` the layer's pool ``[slots, Hkv, D]``; prefix rows
    ``kv_indices[kv_indptr[s]:kv_indptr[s+1]]``; queries causal over their own
    keys.  Supported: bf16, head_dim 64/128, causal, no custom mask, no logit
    cap, unit K/V scales; anything else raises ``ValueError``.
    """
    use_context_positions = context_q_positions is not None
    if use_context_positions != (context_kv_positions is not None):
        raise ValueError("Context attention requires both query and KV positions")
    if use_context_positions:
        if page_size != 1:
            raise ValueError("Context attention requires page_size=1")
        for positions, count in ((context_q_positions, q_extend.shape[0]),
                                 (context_kv_positions, kv_indices.numel())):
            if (positions.device != q_extend.device or positions.ndim != 1 or positions.numel() != count
                    or positions.dtype not in (torch.int32, torch.int64) or not positions.is_contiguous()):
                raise ValueError("Context attention positions must align with Q/KV")
        if context_q_positions.dtype != context_kv_positions.dtype:
            raise ValueError("Context attention positions must share one dtype")
    if custom_mask is not None or mask_indptr is not None or not is_causal:
        raise ValueError("only causal extend attention without a custom mask is supported")
    if logit_cap or k_scale != 1.0 or v_scale != 1.0 or window_kv_offsets is not None or xai_temperature_len > 0:
        raise ValueError("logit caps, KV scales, window KV offsets and temperature scaling are not supported")
    for t in (q_extend, k_extend, v_extend, k_buffer, v_buffer):
        if t.dtype != torch.bfloat16 or t.ndim != 3 or t.stride(-1) != 1:
            raise ValueError("q/k/v and the KV pool must be bf16 [tokens, heads, head_dim] with unit dim stride")
    if o_extend.dtype not in (torch.bfloat16, torch.float32) or o_extend.shape != q_extend.shape \
            or o_extend.stride(-1) != 1:
        raise ValueError("o_extend must be bf16 or f32 shaped like q_extend")
    if k_extend.shape[0] != q_extend.shape[0] or v_extend.shape != k_extend.shape \
            or k_buffer.shape[1:] != k_extend.shape[1:] or v_buffer.shape[1:] != k_extend.shape[1:]:
        raise ValueError("k/v extend and the KV pool must share [kv_heads, head_dim]")
    if q_extend.shape[2] != k_extend.shape[2]:
        raise ValueError("q and K head dims differ")
    if qo_indptr.dtype != kv_indptr.dtype or qo_indptr.dtype not in _INDEX or kv_indices.dtype not in _INDEX:
        raise ValueError("indptrs must share an int32/int64 dtype; kv_indices int32 or int64")
    if qo_indptr.ndim != 1 or kv_indptr.shape != qo_indptr.shape:
        raise ValueError("qo_indptr and kv_indptr must be [segments + 1]")
    n_seg = qo_indptr.numel() - 1
    d = q_extend.shape[2]
    scale = sm_scale if sm_scale is not None else d ** -0.5
    if sinks is not None and (sinks.dtype != torch.float32 or sinks.shape != (q_extend.shape[1],)):
        raise ValueError("sinks must be f32 [q_heads]")
    lib = _lib.load()
    pos_dtype = _INDEX[context_q_positions.dtype] if use_context_positions else _lib.AKV_I64
    with _on_device(q_extend.device):
        rc = lib.akv_context_attention(
            q_extend.data_ptr(), q_extend.stride(0), q_extend.stride(1),
            k_extend.data_ptr(), v_extend.data_ptr(), k_extend.stride(0), k_extend.stride(1),
            v_extend.stride(0), v_extend.stride(1),
            k_buffer.data_ptr(), v_buffer.data_ptr(), k_buffer.stride(0), k_buffer.stride(1),
            v_buffer.stride(0), v_buffer.stride(1),
            n_seg, q_extend.shape[1], k_extend.shape[1], d,
            qo_indptr.data_ptr(), kv_indptr.data_ptr(), _INDEX[qo_indptr.dtype],
            kv_indices.data_ptr() if kv_indices.numel() else None, _INDEX[kv_indices.dtype],
            _lib.ptr(context_q_positions), _lib.ptr(context_kv_positions), pos_dtype,
            int(sliding_window_size) if sliding_window_size is not None else -1,
            _lib.ptr(sinks), float(scale), o_extend.data_ptr(),
            _lib.AKV_F32 if o_extend.dtype == torch.float32 else _lib.AKV_BF16,
            o_extend.stride(0), o_extend.stride(1), int(max_len_extend),
            current_stream_handle(q_extend.device),
        )
    _lib.check(rc, "akv_context_attention")
    return o_extend
