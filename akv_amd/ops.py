"""Drop-in ``reposition_kv_layers`` on the gfx950 HIP kernel.

Same signature, argument meaning, validation order and ``ValueError``
messages as the reference wrapper
(``akv/system/sglang/kernels/ops/attention/context_reposition.py:126-236``);
the launch goes to ``akv_reposition_kv_layers`` in ``libakv_amd.so`` on the
current HIP stream of the KV device.  No allocation, no device-to-host read,
no synchronisation.
"""

import torch

from . import _lib

_KV_DTYPES = {torch.float32: _lib.AKV_F32, torch.float16: _lib.AKV_F16, torch.bfloat16: _lib.AKV_BF16}


def current_stream_handle(device):
    """hipStream_t of torch's current stream on ``device``, as an int."""
    return torch.cuda.current_stream(device).cuda_stream


class _on_device:
    """Makes ``device`` current for the duration of a launch (cheap when it already is)."""

    __slots__ = ("index", "previous")

    def __init__(self, device):
        self.index = device.index if device.index is not None else torch.cuda.current_device()
        self.previous = None

    def __enter__(self):
        current = torch.cuda.current_device()
        if current != self.index:
            self.previous = current
            torch.cuda.set_device(self.index)
        return self

    def __exit__(self, *exc):
        if self.previous is not None:
            torch.cuda.set_device(self.previous)
        return False


def reposition_kv_layers(
    k_data_ptrs: torch.Tensor,
    v_data_ptrs: torch.Tensor,
    k_layout: torch.Tensor,
    v_layout: torch.Tensor,
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    position_pairs: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    *,
    is_neox_style: bool = True,
    page_size: int = 1,
    skip_unmapped: bool = False,
    rotary_dim: int | None = None,
) -> None:
    """Rotate K and copy V across native per-layer pools in one GPU launch.

    ``k_data_ptrs``/``v_data_ptrs`` are device tables of per-layer base
    addresses; every layer shares the exemplar ``k_layout``/``v_layout``
    dtype and NHD strides.  For each moved token, K's rotary part goes from
    ``position_pairs[t, 0]`` to ``position_pairs[t, 1]`` and K's tail and V
    are copied, from ``source_slots[t]`` to ``destination_slots[t]``.

    The caller owns fresh destination slots disjoint from all sources and
    keeps the sources and metadata alive until the stream finishes.  This
    wrapper does no GPU-to-CPU read and no synchronisation, and allocates no
    KV page.
    """
    _reposition(k_data_ptrs, v_data_ptrs, k_layout, v_layout, source_slots, destination_slots, position_pairs,
                cos_sin_cache, is_neox_style, page_size, skip_unmapped, rotary_dim, None)


def reposition_kv_layers_gated(
    k_data_ptrs: torch.Tensor,
    v_data_ptrs: torch.Tensor,
    k_layout: torch.Tensor,
    v_layout: torch.Tensor,
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    position_pairs: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    *,
    status: torch.Tensor,
    is_neox_style: bool = True,
    page_size: int = 1,
    skip_unmapped: bool = False,
    rotary_dim: int | None = None,
) -> None:
    """``reposition_kv_layers`` behind the device status word of the
    compaction that built the lists (``tables.compact_rows``'s
    ``outputs.status``): every workgroup reads it and, when the lists are
    unusable, touches no K/V row and writes nothing.  So the lists go from
    the compaction to the Reposition on one stream with no host read."""
    if status.dtype != torch.int32 or status.numel() < 1 or status.device != k_layout.device:
        raise ValueError("status must be an int32 device word on the KV device")
    _reposition(k_data_ptrs, v_data_ptrs, k_layout, v_layout, source_slots, destination_slots, position_pairs,
                cos_sin_cache, is_neox_style, page_size, skip_unmapped, rotary_dim, status)


def _reposition(k_data_ptrs, v_data_ptrs, k_layout, v_layout, source_slots, destination_slots, position_pairs,
                cos_sin_cache, is_neox_style, page_size, skip_unmapped, rotary_dim, status):
    if page_size != 1:
        raise ValueError("Context Reposition requires page_size=1")
    tensors = (
        k_data_ptrs,
        v_data_ptrs,
        k_layout,
        v_layout,
        source_slots,
        destination_slots,
        position_pairs,
        cos_sin_cache,
    )
    if not k_layout.is_cuda or any(t.device != k_layout.device for t in tensors):
        raise ValueError("Reposition tensors must be on one CUDA device")
    if k_layout.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("Context Reposition requires unquantized floating-point KV")
    if (
        k_layout.ndim != 3
        or v_layout.shape != k_layout.shape
        or v_layout.dtype != k_layout.dtype
    ):
        raise ValueError("Reposition requires matching native NHD K/V layouts")
    if k_layout.stride(-1) != 1 or v_layout.stride(-1) != 1:
        raise ValueError("Reposition requires contiguous head dimensions")
    if (
        k_data_ptrs.ndim != 1
        or v_data_ptrs.shape != k_data_ptrs.shape
        or k_data_ptrs.dtype not in (torch.uint64, torch.int64)
        or v_data_ptrs.dtype not in (torch.uint64, torch.int64)
        or not k_data_ptrs.is_contiguous()
        or not v_data_ptrs.is_contiguous()
    ):
        raise ValueError("Reposition requires contiguous 64-bit layer pointer tables")
    count = len(source_slots)
    if (
        source_slots.ndim != 1
        or destination_slots.shape != source_slots.shape
        or source_slots.dtype != torch.int32
        or destination_slots.dtype != torch.int32
        or not source_slots.is_contiguous()
        or not destination_slots.is_contiguous()
        or position_pairs.shape != (count, 2)
        or position_pairs.dtype != torch.int32
        or position_pairs.stride(-1) != 1
    ):
        raise ValueError("Reposition requires int32 slot vectors and [N, 2] positions")
    head_dim = k_layout.shape[-1]
    rotary_dim = head_dim if rotary_dim is None else rotary_dim
    if (
        type(rotary_dim) is not int
        or not 0 < rotary_dim <= head_dim
        or rotary_dim % 2
        or cos_sin_cache.ndim != 2
        or cos_sin_cache.shape[1] != rotary_dim
        or cos_sin_cache.stride(-1) != 1
        or not cos_sin_cache.is_floating_point()
    ):
        raise ValueError("Reposition requires a native cos/sin cache matching rotary_dim")
    if count == 0 or len(k_data_ptrs) == 0:
        return
    table_dtype = _KV_DTYPES.get(cos_sin_cache.dtype)
    if table_dtype is None:
        raise ValueError("Reposition cos/sin cache must be float32, float16 or bfloat16")
    lib = _lib.load()
    with _on_device(k_layout.device):
        rc = lib.akv_reposition_kv_layers_gated(
            k_data_ptrs.data_ptr(),
            v_data_ptrs.data_ptr(),
            len(k_data_ptrs),
            _KV_DTYPES[k_layout.dtype],
            k_layout.shape[1],
            head_dim,
            rotary_dim,
            k_layout.stride(0),
            k_layout.stride(1),
            v_layout.stride(0),
            v_layout.stride(1),
            source_slots.data_ptr(),
            destination_slots.data_ptr(),
            position_pairs.data_ptr(),
            position_pairs.stride(0),
            count,
            cos_sin_cache.data_ptr(),
            table_dtype,
            cos_sin_cache.stride(0),
            1 if is_neox_style else 0,
            1 if skip_unmapped else 0,
            _lib.ptr(status),
            current_stream_handle(k_layout.device),
        )
    _lib.check(rc, "akv_reposition_kv_layers")
