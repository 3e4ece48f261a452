"""CPU restatement of the all-layer Reposition (K re-rotation + V move).

Follows ``_reposition_layers_kernel``
(``akv/system/sglang/kernels/ops/attention/context_reposition.py:54-123``):

* slots are read as int64; with ``skip_unmapped`` a token whose source or
  destination slot is ``<= 0`` is left alone (``:58-62``);
* pairs are ``(i, i + R/2)`` for NeoX style and ``(2i, 2i + 1)`` otherwise
  (``:77-80``); cos is ``cache[pos, 0:R/2]``, sin ``cache[pos, R/2:R]``
  (``:82-91``), both read as fp32;
* in fp32, every product and sum rounded on its own (no FMA,
  ``enable_fp_fusion=False`` at ``:235``), with IEEE division (``tl.div_rn``)::

      s  = (co*co) + (so*so)
      u1 = ((x1*co) + (x2*so)) / s
      u2 = ((x2*co) - (x1*so)) / s
      y1 = (u1*cn) - (u2*sn)
      y2 = (u2*cn) + (u1*sn)                                  (:92-102)

* when ``old == new`` the original bits are stored (``:98-112``);
* results are narrowed with round-to-nearest-even (Triton's downcast);
* K dims ``[R, D)`` and all of V are copied bit for bit (``:114-123``).

Pinned by (``tests/test_oracle_reposition.py``):

* 64 known answers on the GPT-OSS YaRN table
  (``tests/golden/reposition_kat.npz``) whose expected bf16 bits come from
  exact rational arithmetic with fp32 round-to-nearest-even after every
  operation (``tests/exact_fp.py``).  Each case was chosen so that a
  delta-angle rotation, division of each product before the sum, and fused
  multiply-adds all give different bits; the test plants each of those forms
  in place of ``rotate_pairs`` and checks that the known answers reject it;
* rotation by quarter turns (tables with cos/sin in {-m, 0, m}) against the
  closed forms (x1, x2) -> (-x2, x1) / (x2, -x1), which catch a swapped sign,
  a cos/sin half swap, a wrong pair index or a missing division;
* ``old == new`` -> bits unchanged; plain-RoPE round trips p -> q -> p
  within 2 bf16 ulp; a float64 delta rotation within 2^-6 of the pair;
* bitwise V/tail copies, and ``skip_unmapped`` leaving the destination
  untouched.

Non-finite inputs follow IEEE-754: infinities propagate through the same
operations, and a NaN input or an invalid operation (inf - inf, 0 * inf)
gives a NaN.  A same-position copy keeps the source bits, NaN payloads
included.  The GPU test ``test_nonfinite_inputs`` holds the kernel to this
bit for bit wherever the result is not a NaN, and to NaN exactly where this
restatement has one.  Parity unpinned: the payload of a NaN that the
rotation produces; each machine's arithmetic picks its own.
"""

import numpy as np

from .bf16 import from_f32, to_f32


def _pair_index(rotary_dim, is_neox_style):
    half = rotary_dim // 2
    i = np.arange(half)
    if is_neox_style:
        return i, i + half
    return 2 * i, 2 * i + 1


def rotate_pairs(x1, x2, co, so, cn, sn):
    """The fp32 two-step rotation, every operation rounded separately."""
    f = np.float32
    x1, x2 = x1.astype(f), x2.astype(f)
    co, so, cn, sn = (a.astype(f) for a in (co, so, cn, sn))
    s = (co * co) + (so * so)
    u1 = ((x1 * co) + (x2 * so)) / s
    u2 = ((x2 * co) - (x1 * so)) / s
    y1 = (u1 * cn) - (u2 * sn)
    y2 = (u2 * cn) + (u1 * sn)
    return y1.astype(f), y2.astype(f)


def reposition_kv_layers(
    k_layers,
    v_layers,
    source_slots,
    destination_slots,
    position_pairs,
    cos_sin_cache,
    *,
    dtype,
    cos_sin_dtype="f32",
    is_neox_style=True,
    skip_unmapped=False,
    rotary_dim=None,
):
    """Apply one Reposition to numpy copies of per-layer KV buffers, in place.

    ``k_layers``/``v_layers``: lists of ``[S, H, D]`` storage arrays (uint16
    bit patterns for 'bf16'/'f16', float32 for 'f32').  ``position_pairs`` is
    ``[M, 2]`` (old, new).  ``cos_sin_cache`` is ``[P, R]`` storage of
    ``cos_sin_dtype``.
    """
    src = np.asarray(source_slots, dtype=np.int64)
    dst = np.asarray(destination_slots, dtype=np.int64)
    pairs = np.asarray(position_pairs, dtype=np.int64).reshape(-1, 2)
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
    table = to_f32(cos_sin_cache, cos_sin_dtype).reshape(cos_sin_cache.shape)
    co, so = table[old, :half], table[old, half:rotary_dim]
    cn, sn = table[new, :half], table[new, half:rotary_dim]
    co, so, cn, sn = (a[:, None, :] for a in (co, so, cn, sn))
    same = (old == new)[:, None, None]
    first, second = _pair_index(rotary_dim, is_neox_style)
    for k, v in zip(k_layers, v_layers):
        rows = k[src].copy()  # [M, H, D] storage
        x1 = to_f32(rows[..., first], dtype).reshape(rows[..., first].shape)
        x2 = to_f32(rows[..., second], dtype).reshape(rows[..., second].shape)
        y1, y2 = rotate_pairs(x1, x2, co, so, cn, sn)
        out = rows.copy()
        b1 = from_f32(y1, dtype).reshape(y1.shape)
        b2 = from_f32(y2, dtype).reshape(y2.shape)
        out[..., first] = np.where(same, rows[..., first], b1)
        out[..., second] = np.where(same, rows[..., second], b2)
        # dims [R, D) of K already hold the source bits (bitwise tail copy)
        k[dst] = out
        v[dst] = v[src]


def algorithmic_bytes(moved, n_layers, n_heads, head_dim, kv_bytes, rotary_dim, table_bytes=4):
    """HBM bytes one Reposition must move (K/V read+write, slot lists, tables)."""
    kv = moved * 4 * n_layers * n_heads * head_dim * kv_bytes
    meta = moved * 16
    rope = moved * 2 * rotary_dim * table_bytes
    return kv, kv + meta + rope
