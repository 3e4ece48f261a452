"""Pins oracle.attention against torch SDPA and the reference's sink formula."""

import numpy as np
import torch

from oracle import attention as at


def test_no_sink_equals_sdpa():
    rng = np.random.default_rng(0)
    hq, hkv, d, n = 16, 4, 64, 37
    q = rng.standard_normal((hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    got = at.decode_attention(q, k, v, 0.125)
    kk = torch.from_numpy(k).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)  # [hq, n, d]
    vv = torch.from_numpy(v).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[:, None, :], kk, vv, scale=0.125)[:, 0, :]
    np.testing.assert_allclose(got, want.numpy(), atol=2e-6, rtol=1e-5)


def test_sink_equals_sigmoid_of_lse_form():
    rng = np.random.default_rng(1)
    hq, hkv, d, n = 8, 8, 32, 100
    q = rng.standard_normal((hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    sinks = rng.standard_normal(hq).astype(np.float32) * 3
    got = at.decode_attention(q, k, v, 0.2, sinks)
    base = at.decode_attention(q, k, v, 0.2)
    s = 0.2 * np.einsum("nhd,hd->hn", k.astype(np.float64), q.astype(np.float64))
    lse = torch.logsumexp(torch.from_numpy(s), dim=1).numpy()
    want = base * torch.sigmoid(torch.from_numpy(lse - sinks)).numpy()[:, None]
    np.testing.assert_allclose(got, want, atol=1e-6, rtol=1e-5)


def test_single_key_closed_form():
    q = np.array([[1.0, 2.0]], dtype=np.float32)
    k = np.array([[[0.5, 0.25]]], dtype=np.float32)
    v = np.array([[[3.0, -1.0]]], dtype=np.float32)
    s = 1.0 * (0.5 + 0.5)
    want = v[0, 0] * np.exp(s) / (np.exp(s) + np.exp(0.3))
    np.testing.assert_allclose(at.decode_attention(q, k, v, 1.0, np.array([0.3]))[0], want, rtol=1e-6)
    assert np.all(at.decode_attention(q, k[:0], v[:0], 1.0, np.array([0.3])) == 0)
