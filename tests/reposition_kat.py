"""Known answers of the Reposition's fp32 rotation (tests/golden/reposition_kat.npz).

64 (x1, x2, old, new) cases on the GPT-OSS YaRN table whose bf16 result under
the reference order (context_reposition.py:92-102, every operation rounded,
no FMA) differs from a delta-angle rotation, from dividing each product
before the sum and from fused multiply-adds.  The expected bits come from
exact rational arithmetic (tests/exact_fp.py); the fixture is written by
tests/golden/make_reposition_kat.py.
"""

from pathlib import Path

import numpy as np

KAT = np.load(Path(__file__).resolve().parent / "golden" / "reposition_kat.npz")
KAT_VARIANTS = ("delta_angle", "per_term_division", "fused")


def kat_pool(neox=True, dim=64):
    """One token per case: every rotary pair of its K row holds the case's
    (x1, x2); table rows 2c / 2c + 1 hold the case's old / new cos|sin in
    every frequency.  Returns (k, v, src, dst, pairs, table)."""
    n = len(KAT["old"])
    half = dim // 2
    k = np.zeros((1 + 2 * n, 1, dim), dtype=np.uint16)
    v = np.zeros_like(k)
    first, second = (np.arange(half), np.arange(half) + half) if neox else \
        (2 * np.arange(half), 2 * np.arange(half) + 1)
    k[1 : n + 1, 0][:, first] = KAT["x1_bits"][:, None]
    k[1 : n + 1, 0][:, second] = KAT["x2_bits"][:, None]
    v[1 : n + 1] = (np.arange(n * dim, dtype=np.uint16) % 30000 + 1).reshape(n, 1, dim)
    table = np.zeros((2 * n, dim), dtype=np.uint32)
    table[0::2, :half] = KAT["co_bits"][:, None]
    table[0::2, half:] = KAT["so_bits"][:, None]
    table[1::2, :half] = KAT["cn_bits"][:, None]
    table[1::2, half:] = KAT["sn_bits"][:, None]
    pairs = np.stack((np.arange(0, 2 * n, 2), np.arange(1, 2 * n, 2)), 1)
    return [k], [v], np.arange(1, n + 1), np.arange(n + 1, 2 * n + 1), pairs, table.view(np.float32)


def kat_expected(form="two_step", neox=True, dim=64):
    half = dim // 2
    want = np.zeros((len(KAT["old"]), 1, dim), dtype=np.uint16)
    first, second = (np.arange(half), np.arange(half) + half) if neox else \
        (2 * np.arange(half), 2 * np.arange(half) + 1)
    want[:, 0][:, first] = KAT[f"{form}_bits"][:, 0:1]
    want[:, 0][:, second] = KAT[f"{form}_bits"][:, 1:2]
    return want
