"""Pins oracle.bf16 against torch's RNE casts and hand-built halfway cases."""

import numpy as np
import torch

from oracle import bf16


def _torch_bf16_bits(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_halfway_cases_round_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1.0 + 2^-7: ties go to even (1.0)
    # 1 + 3*2^-8 is halfway between 1+2^-7 (odd) and 1+2^-6: ties go to 1+2^-6
    cases = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 1 + 2**-8 + 2**-20], dtype=np.float32)
    got = bf16.f32_to_bf16_bits(cases)
    want = np.array([0x3F80, 0x3F82, 0xBF80, 0x3F81], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)
    # truncation would give 0x3F81 for the second case and round-half-up 0x3F81 for the first
    np.testing.assert_array_equal(got, _torch_bf16_bits(cases))


def test_specials_and_subnormals():
    x = np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -3e-39, 3.3895314e38, 1e-45], dtype=np.float32)
    np.testing.assert_array_equal(bf16.f32_to_bf16_bits(x), _torch_bf16_bits(x))
    # largest finite values round to infinity when above the bf16 max + half ulp
    big = np.array([3.4028235e38], dtype=np.float32)
    assert bf16.f32_to_bf16_bits(big)[0] == 0x7F80


def test_random_against_torch():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    np.testing.assert_array_equal(bf16.f32_to_bf16_bits(x), _torch_bf16_bits(x))


def test_nan_stays_nan():
    out = bf16.bf16_bits_to_f32(bf16.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32)))
    assert np.isnan(out[0])


def test_f16_and_roundtrip():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(10000).astype(np.float32)
    np.testing.assert_array_equal(
        bf16.f32_to_f16_bits(x), torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    )
    b = bf16.f32_to_bf16_bits(x)
    np.testing.assert_array_equal(bf16.f32_to_bf16_bits(bf16.bf16_bits_to_f32(b)), b)
