"""IEEE-754 narrowing used by every store of the Reposition kernel.

The reference stores fp32 results into bf16/fp16 KV with Triton's default
downcast, which is round-to-nearest-even
(``akv/system/sglang/kernels/ops/attention/context_reposition.py:103-112``).

Pinned by: exhaustive agreement with ``torch.Tensor.to(torch.bfloat16)`` /
``numpy.float16`` on hand-picked halfway cases, signed zeros, subnormals,
infinities and a large random sample (``tests/test_oracle_bf16.py``); the
halfway cases are chosen so that round-half-up or truncation fail.
"""

import numpy as np


def f32_to_bf16_bits(x):
    """fp32 array -> uint16 bf16 bit patterns, round-to-nearest-even.

    NaN inputs become a quiet NaN with the sign and top payload bits kept.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    rounded = ((u + 0x7FFF + lsb) >> 16) & 0xFFFF
    nan = np.isnan(x)
    if nan.any():
        quiet = ((u >> 16) | 0x0040) & 0xFFFF
        rounded = np.where(nan, quiet, rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits):
    """uint16 bf16 bit patterns -> fp32 (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def f32_to_f16_bits(x):
    """fp32 -> IEEE binary16 bits, round-to-nearest-even (numpy's cast is RNE)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return x.astype(np.float16).view(np.uint16)


def f16_bits_to_f32(bits):
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_f32(bits_or_values, dtype):
    """Storage array of ``dtype`` ('bf16', 'f16', 'f32') -> fp32 values."""
    if dtype == "bf16":
        return bf16_bits_to_f32(bits_or_values)
    if dtype == "f16":
        return f16_bits_to_f32(bits_or_values)
    if dtype == "f32":
        return np.ascontiguousarray(bits_or_values).view(np.float32).astype(np.float32)
    raise ValueError(dtype)


def from_f32(values, dtype):
    """fp32 values -> storage array of ``dtype`` (uint16 bits or float32)."""
    if dtype == "bf16":
        return f32_to_bf16_bits(values)
    if dtype == "f16":
        return f32_to_f16_bits(values)
    if dtype == "f32":
        return np.ascontiguousarray(values, dtype=np.float32)
    raise ValueError(dtype)
