"""Prefill context attention (host side of ``akv_context_attention``).

``extend_attention_fwd`` is the drop-in for the extend-attention entry with
context positions (``akv/system/sglang.patch:106-237``): same arguments,
checks and messages.  The reference's prefill metadata builder
(``context_backend.py:24-251``) passes it qo/kv indptrs, the bound prefix
slots and the query / key positions unchanged.  The device work is
``akv_context_attention`` in ``libakv_amd.so``; there is no other path.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .ops import _on_device, current_stream_handle


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
    keys.  Supported: bf16 inputs, bf16 or f32 output, head dims that are
    multiples of 8 up to 128, any GQA group of up to 128 q heads per KV
    head, logit caps (``cap * tanh(score / cap)``), row strides that are
    multiples of 8 elements, causal, no custom mask, unit K/V scales;
    anything else raises ``ValueError`` (the reference's Triton kernel also
    takes wider heads, Q/K and V heads of different widths, custom masks and
    KV scales).
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
    if k_scale != 1.0 or v_scale != 1.0 or window_kv_offsets is not None or xai_temperature_len > 0:
        raise ValueError("KV scales, window KV offsets and temperature scaling are not supported")
    if logit_cap is None or not logit_cap >= 0.0 or logit_cap == float("inf"):
        raise ValueError("logit_cap must be 0 (no cap) or positive and finite")
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
            _lib.ptr(sinks), float(scale), float(logit_cap), o_extend.data_ptr(),
            _lib.AKV_F32 if o_extend.dtype == torch.float32 else _lib.AKV_BF16,
            o_extend.stride(0), o_extend.stride(1), int(max_len_extend),
            current_stream_handle(q_extend.device),
        )
    _lib.check(rc, "akv_context_attention")
    return o_extend
