"""torch-CPU restatement of the Reposition, vectorised -- the CPU baseline.

The same arithmetic as ``oracle.reposition`` (which follows
``akv/system/sglang/kernels/ops/attention/context_reposition.py:54-123``),
written with torch CPU tensor operations over ``[layers, moved, heads,
rotary_dim / 2]`` so that it runs on every host core: the baseline that the
GPU is timed against.  Every fp32 product, sum and quotient is its own eager
torch operation, so each is rounded on its own (no fused multiply-add), the
quotient is IEEE division, and the narrowing to bf16/fp16 is torch's
round-to-nearest-even cast.

    s  = (co*co) + (so*so)
    u1 = ((x1*co) + (x2*so)) / s
    u2 = ((x2*co) - (x1*so)) / s
    y1 = (u1*cn) - (u2*sn)
    y2 = (u2*cn) + (u1*sn)                                  (:92-102)

A token whose old and new positions are equal keeps its source bits
(``:98-112``); K dims ``[R, D)`` and all of V are copied bit for bit
(``:114-123``).

Pinned by (``tests/test_oracle_cpu_torch.py``): the exact-arithmetic known
answers of ``tests/golden/reposition_kat.npz`` (the same ones that pin
``oracle.reposition``), and bit-for-bit agreement with ``oracle.reposition``
on random pools across dtypes, NeoX / GPT-J pairs, partial rotary widths,
same-position tokens and ``skip_unmapped``.

Test infrastructure only (see the package docstring).
"""

import torch


def _pair_index(rotary_dim, is_neox_style):
    half = rotary_dim // 2
    i = torch.arange(half)
    if is_neox_style:
        return i, i + half
    return 2 * i, 2 * i + 1


def reposition_kv_layers(k_layers, v_layers, source_slots, destination_slots, position_pairs, cos_sin_cache, *,
                         is_neox_style=True, skip_unmapped=False, rotary_dim=None):
    """One Reposition over CPU torch KV buffers, in place.

    ``k_layers`` / ``v_layers``: lists of ``[S, H, D]`` CPU tensors (bf16,
    fp16 or fp32); ``source_slots`` / ``destination_slots``: integer ``[M]``;
    ``position_pairs``: ``[M, 2]`` (old, new); ``cos_sin_cache``: ``[P, R]``
    (cos | sin) of any float dtype, read as fp32.
    """
    src = torch.as_tensor(source_slots).to(torch.int64)
    dst = torch.as_tensor(destination_slots).to(torch.int64)
    pairs = torch.as_tensor(position_pairs).to(torch.int64).reshape(-1, 2)
    if len(src) == 0 or len(k_layers) == 0:
        return
    head_dim = k_layers[0].shape[-1]
    rotary_dim = head_dim if rotary_dim is None else rotary_dim
    half = rotary_dim // 2
    if skip_unmapped:
        live = (src > 0) & (dst > 0)
        src, dst, pairs = src[live], dst[live], pairs[live]
        if len(src) == 0:
            return
    old, new = pairs[:, 0], pairs[:, 1]
    table = cos_sin_cache.to(torch.float32)
    # [1, M, 1, half]: one coefficient per (token, frequency), every layer and head
    co = table[old, :half][None, :, None, :]
    so = table[old, half:rotary_dim][None, :, None, :]
    cn = table[new, :half][None, :, None, :]
    sn = table[new, half:rotary_dim][None, :, None, :]
    same = (old == new)[None, :, None, None]
    first, second = _pair_index(rotary_dim, is_neox_style)

    rows = torch.stack([k[src] for k in k_layers])  # [L, M, H, D] storage
    x1 = rows[..., first].to(torch.float32)
    x2 = rows[..., second].to(torch.float32)
    s = torch.add(torch.mul(co, co), torch.mul(so, so))
    u1 = torch.div(torch.add(torch.mul(x1, co), torch.mul(x2, so)), s)
    u2 = torch.div(torch.sub(torch.mul(x2, co), torch.mul(x1, so)), s)
    y1 = torch.sub(torch.mul(u1, cn), torch.mul(u2, sn)).to(rows.dtype)
    y2 = torch.add(torch.mul(u2, cn), torch.mul(u1, sn)).to(rows.dtype)
    out = rows.clone()
    out[..., first] = torch.where(same, rows[..., first], y1)
    out[..., second] = torch.where(same, rows[..., second], y2)
    for layer, (k, v) in enumerate(zip(k_layers, v_layers)):
        k[dst] = out[layer]
        v[dst] = v[src]
