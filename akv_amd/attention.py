"""GQA decode attention with sinks over compacted indices (HIP, MFMA).

The consumer of the Drop + Reposition metadata: one decode step per layer
reading each request's keys through ``kv_indptr`` / ``kv_indices`` (a full
layer's compacted rows from ``compact_rows`` / ``ContextDecodeRegistry.fill``,
or a sliding-window layer's from ``fill_window``), normalised with per-head
sink logits exactly as the reference's ``o * sigmoid(lse - sink)``
(``akv/system/sglang/srt/layers/attention/context_backend.py:254-272``).
"""

import torch

from . import _lib
from .ops import _on_device, current_stream_handle


def workspace_bytes(n_requests, kv_heads, head_dim, max_len):
    return _lib.load().akv_decode_attention_workspace_bytes(n_requests, kv_heads, head_dim, max_len)


def decode_attention(q, k_buffer, v_buffer, kv_indptr, kv_indices, out, *, scale, max_len, sinks=None,
                     workspace=None, status=None):
    """``out[b, h] = softmax-with-sink(scale * q[b, h] . K_j) . V_j`` over request b's indices.

    ``q``/``out``: ``[B, q_heads, D]`` (bf16 q; bf16 or f32 out); ``k_buffer``/
    ``v_buffer``: one layer's ``[slots, kv_heads, D]`` bf16 pool; ``kv_indptr``
    int32 ``[B+1]``; ``kv_indices`` int32; ``sinks`` f32 ``[q_heads]``;
    ``max_len``: host bound on every request's key count.  ``status``: the
    compaction's device status word when the indices come from it (the
    kernels then skip their work on the device when it reports them
    unusable).
    """
    if q.dtype != torch.bfloat16 or q.ndim != 3 or q.stride(-1) != 1:
        raise ValueError("q must be bf16 [B, q_heads, head_dim] with unit dim stride")
    if (k_buffer.dtype != torch.bfloat16 or v_buffer.dtype != torch.bfloat16 or k_buffer.ndim != 3
            or v_buffer.shape != k_buffer.shape or k_buffer.stride(-1) != 1 or v_buffer.stride(-1) != 1):
        raise ValueError("K/V must be matching bf16 [slots, kv_heads, head_dim] buffers")
    if out.dtype not in (torch.bfloat16, torch.float32) or out.shape != q.shape or out.stride(-1) != 1:
        raise ValueError("out must be bf16 or f32 shaped like q")
    if kv_indptr.dtype != torch.int32 or kv_indices.dtype != torch.int32 or len(kv_indptr) != q.shape[0] + 1:
        raise ValueError("kv_indptr / kv_indices must be int32, indptr of length B + 1")
    if sinks is not None and (sinks.dtype != torch.float32 or sinks.shape != (q.shape[1],)):
        raise ValueError("sinks must be f32 [q_heads]")
    if q.shape[2] != k_buffer.shape[2]:
        raise ValueError("q and K head dims differ")
    if status is not None and (status.dtype != torch.int32 or status.numel() < 1 or status.device != q.device):
        raise ValueError("status must be an int32 device word on q's device")
    n, hq, d = q.shape
    hkv = k_buffer.shape[1]
    need = workspace_bytes(n, hkv, d, max_len)
    if workspace is None:
        workspace = torch.empty(max(4, (need + 3) // 4), dtype=torch.float32, device=q.device)
    lib = _lib.load()
    with _on_device(q.device):
        rc = lib.akv_decode_attention(
            q.data_ptr(), q.stride(0), q.stride(1), k_buffer.data_ptr(), v_buffer.data_ptr(),
            k_buffer.stride(0), k_buffer.stride(1), v_buffer.stride(0), v_buffer.stride(1), n, hq, hkv, d,
            kv_indptr.data_ptr(), kv_indices.data_ptr(), _lib.ptr(sinks), float(scale), out.data_ptr(),
            _lib.AKV_F32 if out.dtype == torch.float32 else _lib.AKV_BF16, out.stride(0), out.stride(1),
            int(max_len), workspace.data_ptr(), workspace.numel() * workspace.element_size(), _lib.ptr(status),
            current_stream_handle(q.device),
        )
    _lib.check(rc, "akv_decode_attention")
    return out
