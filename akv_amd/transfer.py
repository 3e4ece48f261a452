"""All-layer KV row copies for the compacted final-version handoff.

The P side packs a request's active rows (``request_active_slots``,
``akv/system/sglang/srt/disaggregation/context_transfer.py:110-128``) into a
contiguous buffer; the D side unpacks them into the owners it allocated
(``allocate_context_destination``, ``:201-259``).  Both, and a direct
pool-to-pool copy (peer pointers on another GPU of the node), are one
``akv_copy_kv_rows`` launch.
"""

from dataclasses import dataclass

import torch

from . import _lib
from .ops import _on_device, current_stream_handle


def _row_layout(t):
    if t.ndim != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2]:
        raise ValueError("KV layers must be [slots, heads, head_dim] with contiguous heads")
    if t.data_ptr() % 16 or (t.stride(0) * t.element_size()) % 16:
        raise ValueError("KV rows must be 16-byte aligned")
    return t.shape[1] * t.shape[2] * t.element_size(), t.stride(0) * t.element_size()


def _slots(s, n, what):
    if s is None:
        return None
    if s.dtype != torch.int32 or s.shape != (n,):
        raise ValueError(f"{what} must be int32 [tokens]")
    return s.data_ptr()


def copy_kv_rows(src_k_ptrs, src_v_ptrs, src_layout, dst_k_ptrs, dst_v_ptrs, dst_layout, n_tokens, *,
                 src_slots=None, dst_slots=None, status=None):
    """Copy K and V rows of every layer: ``dst[dst_slots[t]] = src[src_slots[t]]``.

    ``*_ptrs``: device uint64/int64 ``[layers]`` base addresses; ``*_layout``:
    an exemplar layer tensor giving the row size and slot stride of that side.
    A missing slot vector means slot ``t`` (a packed buffer).  ``status``:
    the compaction's device status word when a slot vector comes from it
    (nothing is copied, on the device, when it reports the lists unusable).
    """
    for p in (src_k_ptrs, src_v_ptrs, dst_k_ptrs, dst_v_ptrs):
        if p.dtype not in (torch.uint64, torch.int64) or p.ndim != 1 or not p.is_contiguous():
            raise ValueError("layer pointer tables must be contiguous 64-bit vectors")
    n_layers = src_k_ptrs.numel()
    if any(p.numel() != n_layers for p in (src_v_ptrs, dst_k_ptrs, dst_v_ptrs)):
        raise ValueError("layer pointer tables differ in length")
    row, src_stride = _row_layout(src_layout)
    drow, dst_stride = _row_layout(dst_layout)
    if row != drow:
        raise ValueError("source and destination rows differ in size")
    if status is not None and (status.dtype != torch.int32 or status.numel() < 1
                               or status.device != src_k_ptrs.device):
        raise ValueError("status must be an int32 device word on the pointer tables' device")
    lib = _lib.load()
    device = src_k_ptrs.device
    with _on_device(device):
        rc = lib.akv_copy_kv_rows(
            src_k_ptrs.data_ptr(), src_v_ptrs.data_ptr(), dst_k_ptrs.data_ptr(), dst_v_ptrs.data_ptr(), n_layers, row,
            src_stride, src_stride, dst_stride, dst_stride, _slots(src_slots, n_tokens, "src_slots"),
            _slots(dst_slots, n_tokens, "dst_slots"), int(n_tokens), _lib.ptr(status), current_stream_handle(device),
        )
    _lib.check(rc, "akv_copy_kv_rows")


@dataclass
class PackedKV:
    """Contiguous ``[layers, tokens, heads, head_dim]`` K and V of active rows."""

    k: torch.Tensor
    v: torch.Tensor
    k_ptrs: torch.Tensor
    v_ptrs: torch.Tensor

    @classmethod
    def empty(cls, n_layers, n_tokens, heads, head_dim, dtype, device):
        k = torch.empty((n_layers, n_tokens, heads, head_dim), dtype=dtype, device=device)
        v = torch.empty_like(k)
        stride = n_tokens * heads * head_dim * k.element_size()
        base = torch.arange(n_layers, dtype=torch.int64) * stride
        return cls(k, v, (base + k.data_ptr()).to(device), (base + v.data_ptr()).to(device))


def pack_active_kv(k_ptrs, v_ptrs, layout, active_slots, packed):
    """P side: gather the active rows of every layer into ``packed``."""
    copy_kv_rows(k_ptrs, v_ptrs, layout, packed.k_ptrs, packed.v_ptrs, packed.k[0], active_slots.numel(),
                 src_slots=active_slots)


def unpack_active_kv(packed, k_ptrs, v_ptrs, layout, destination_slots):
    """D side: scatter the received rows into the allocated owners."""
    copy_kv_rows(packed.k_ptrs, packed.v_ptrs, packed.k[0], k_ptrs, v_ptrs, layout, destination_slots.numel(),
                 dst_slots=destination_slots)
