"""Writes ``tests/golden/reposition_kat.npz``: known answers for the
Reposition's fp32 rotation that tell its operation order apart from close
mis-statements.

The reference rotates each K pair in fp32 with every operation rounded on its
own (``enable_fp_fusion=False``):
``s = co*co + so*so; u1 = (x1*co + x2*so) / s; u2 = (x2*co - x1*so) / s;
y1 = u1*cn - u2*sn; y2 = u2*cn + u1*sn``, then narrows to bf16 with
round-to-nearest-even
(akv/system/sglang/kernels/ops/attention/context_reposition.py:92-112, :235).

Search: bf16 pairs ~ N(0, 1) and (old, new, frequency) drawn over the
GPT-OSS-120B YaRN table (theta 150000, factor 32, original 4096, 64 rotary
dims, 32768 positions); a vectorised float32 pass proposes candidates whose
bf16 result differs between the reference order and each of three variants
(one rotation by the angle difference, each product divided before the sum,
fused multiply-adds); every kept case is then recomputed with exact rational
arithmetic (``tests/exact_fp.py``, fp32 round-to-nearest-even after every
operation) and kept only if the exact reference bits differ from the exact
bits of all three variants.

Run: ``python tests/golden/make_reposition_kat.py`` (CPU, ~1 minute).
"""

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE.parent))

import exact_fp as ex  # noqa: E402
from akv_amd import rope  # noqa: E402

OUT = HERE / "reposition_kat.npz"
CASES = 64
VARIANTS = ("delta_angle", "per_term_division", "fused")


def _bf16_bits(y):
    """float32 array -> bf16 bits, round-to-nearest-even (finite inputs)."""
    u = y.astype(np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def _fma(a, b, c):
    # the float64 product of two floats is exact; the sum rounds once in
    # float64 and once more to float32 (rare double roundings are removed by
    # the exact recheck)
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def _forms_f32(x1, x2, co, so, cn, sn):
    s = co * co + so * so
    u1 = (x1 * co + x2 * so) / s
    u2 = (x2 * co - x1 * so) / s
    out = {"two_step": (u1 * cn - u2 * sn, u2 * cn + u1 * sn)}
    cd = (cn * co + sn * so) / s
    sd = (sn * co - cn * so) / s
    out["delta_angle"] = (x1 * cd - x2 * sd, x2 * cd + x1 * sd)
    p1 = (x1 * co) / s + (x2 * so) / s
    p2 = (x2 * co) / s - (x1 * so) / s
    out["per_term_division"] = (p1 * cn - p2 * sn, p2 * cn + p1 * sn)
    sf = _fma(co, co, so * so)
    f1 = _fma(x1, co, x2 * so) / sf
    f2 = _fma(x2, co, -(x1 * so)) / sf
    out["fused"] = (_fma(f1, cn, -(f2 * sn)), _fma(f2, cn, f1 * sn))
    return out


def main():
    table = rope.make_table("yarn", 64, 32768, base=150000.0, factor=32.0, original_max=4096,
                            beta_fast=32.0, beta_slow=1.0).numpy()
    half = table.shape[1] // 2
    rng = np.random.default_rng(20260)
    cases = []
    seen = set()
    batch = 1 << 21
    while len(cases) < CASES:
        old = rng.integers(0, table.shape[0], batch)
        new = rng.integers(0, table.shape[0], batch)
        dim = rng.integers(0, half, batch)
        xb1 = _bf16_bits(rng.standard_normal(batch).astype(np.float32))
        xb2 = _bf16_bits(rng.standard_normal(batch).astype(np.float32))
        x1 = (xb1.astype(np.uint32) << 16).view(np.float32)
        x2 = (xb2.astype(np.uint32) << 16).view(np.float32)
        co, so = table[old, dim], table[old, half + dim]
        cn, sn = table[new, dim], table[new, half + dim]
        with np.errstate(all="ignore"):
            forms = _forms_f32(x1, x2, co, so, cn, sn)
        bits = {k: (_bf16_bits(a), _bf16_bits(b)) for k, (a, b) in forms.items()}
        ref = bits["two_step"]
        differs = np.ones(batch, dtype=bool)
        for v in VARIANTS:
            differs &= (bits[v][0] != ref[0]) | (bits[v][1] != ref[1])
        differs &= old != new
        for i in np.flatnonzero(differs):
            key = (int(xb1[i]), int(xb2[i]), int(old[i]), int(new[i]), int(dim[i]))
            if key in seen:
                continue
            seen.add(key)
            tb = [int(np.float32(t).view(np.uint32)) for t in (co[i], so[i], cn[i], sn[i])]
            exact = {f: ex.rotate_bf16_bits(f, key[0], key[1], *tb) for f in ex.FORMS}
            if any(e is None for e in exact.values()):
                continue
            if all(exact[v] != exact["two_step"] for v in VARIANTS):
                cases.append((key, tb, exact))
            if len(cases) == CASES:
                break
        print(f"{len(cases)} cases", flush=True)

    arr = lambda f, dt: np.array([f(c) for c in cases], dtype=dt)  # noqa: E731
    np.savez(
        OUT,
        x1_bits=arr(lambda c: c[0][0], np.uint16), x2_bits=arr(lambda c: c[0][1], np.uint16),
        old=arr(lambda c: c[0][2], np.int32), new=arr(lambda c: c[0][3], np.int32),
        dim=arr(lambda c: c[0][4], np.int32),
        co_bits=arr(lambda c: c[1][0], np.uint32), so_bits=arr(lambda c: c[1][1], np.uint32),
        cn_bits=arr(lambda c: c[1][2], np.uint32), sn_bits=arr(lambda c: c[1][3], np.uint32),
        **{f"{f}_bits": np.array([c[2][f] for c in cases], dtype=np.uint16) for f in ex.FORMS},
    )
    print(f"wrote {OUT} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
