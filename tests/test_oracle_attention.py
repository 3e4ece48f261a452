"""Pins oracle.attention against torch SDPA and the reference's sink formula."""

import numpy as np
import pytest
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


def _segments(rng, hq, hkv, d, q_lens, p_lens, slots=300):
    nq = sum(q_lens)
    q = rng.standard_normal((nq, hq, d)).astype(np.float32)
    ke = rng.standard_normal((nq, hkv, d)).astype(np.float32)
    ve = rng.standard_normal((nq, hkv, d)).astype(np.float32)
    kp = rng.standard_normal((slots, hkv, d)).astype(np.float32)
    vp = rng.standard_normal((slots, hkv, d)).astype(np.float32)
    qo = np.concatenate(([0], np.cumsum(q_lens)))
    kv = np.concatenate(([0], np.cumsum(p_lens)))
    idx = rng.integers(0, slots, size=kv[-1])
    return q, ke, ve, kp, vp, qo, kv, idx


def _sdpa(q, k, v, mask, scale):
    """q [n, hq, d], k/v [m, hkv, d], mask [n, m] -> [n, hq, d] via torch SDPA (fp64)."""
    hq, hkv = q.shape[1], k.shape[1]
    qq = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)
    kk = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
    vv = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
    o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=torch.from_numpy(mask), scale=scale)
    return o.permute(1, 0, 2).numpy()


def test_context_no_prefix_is_causal_sdpa():
    rng = np.random.default_rng(3)
    hq, hkv, d = 8, 2, 16
    q, ke, ve, kp, vp, qo, kv, idx = _segments(rng, hq, hkv, d, [5, 1, 12], [0, 0, 0])
    got = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.25)
    for s in range(3):
        a, b = qo[s], qo[s + 1]
        qq = torch.from_numpy(q[a:b].astype(np.float64)).permute(1, 0, 2)
        kk = torch.from_numpy(ke[a:b].astype(np.float64)).permute(1, 0, 2).repeat_interleave(4, 0)
        vv = torch.from_numpy(ve[a:b].astype(np.float64)).permute(1, 0, 2).repeat_interleave(4, 0)
        want = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True, scale=0.25)
        np.testing.assert_allclose(got[a:b], want.permute(1, 0, 2).numpy(), atol=1e-6, rtol=1e-5)


def test_context_prefix_plus_causal_mask():
    rng = np.random.default_rng(4)
    hq, hkv, d = 4, 4, 8
    q, ke, ve, kp, vp, qo, kv, idx = _segments(rng, hq, hkv, d, [7, 3], [10, 4])
    got = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.3)
    for s in range(2):
        a, b, x, y = qo[s], qo[s + 1], kv[s], kv[s + 1]
        n, p = b - a, y - x
        mask = np.zeros((n, p + n), dtype=bool)
        mask[:, :p] = True
        mask[:, p:] = np.tril(np.ones((n, n), dtype=bool))
        want = _sdpa(q[a:b], np.concatenate((kp[idx[x:y]], ke[a:b])), np.concatenate((vp[idx[x:y]], ve[a:b])),
                     mask, 0.3)
        np.testing.assert_allclose(got[a:b], want, atol=1e-6, rtol=1e-5)


def test_context_window_matches_searchsorted_gather():
    # positions with holes (dropped spans): the reference's native plan finds
    # each query's first visible key by searchsorted over the ordered positions
    rng = np.random.default_rng(5)
    hq, hkv, d, W = 4, 2, 8, 6
    q_lens, p_lens = [9, 4], [12, 0]
    q, ke, ve, kp, vp, qo, kv, idx = _segments(rng, hq, hkv, d, q_lens, p_lens)
    kpos = np.concatenate([np.sort(rng.choice(40, size=n, replace=False)) for n in p_lens])
    qpos = np.concatenate([50 + np.sort(rng.choice(30, size=n, replace=False)) for n in q_lens])
    qpos[9:] = np.sort(rng.choice(20, size=4, replace=False))
    got = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.5, window=W, q_positions=qpos,
                               kv_positions=kpos)
    for s in range(2):
        a, b, x, y = qo[s], qo[s + 1], kv[s], kv[s + 1]
        positions = np.r_[kpos[x:y], qpos[a:b]]
        keys_k = np.concatenate((kp[idx[x:y]], ke[a:b]))
        keys_v = np.concatenate((vp[idx[x:y]], ve[a:b]))
        for i in range(b - a):
            end = y - x + i + 1
            start = np.searchsorted(positions[:end], qpos[a + i] - W)
            mask = np.ones((1, end - start), dtype=bool)
            want = _sdpa(q[a + i : a + i + 1], keys_k[start:end], keys_v[start:end], mask, 0.5)
            np.testing.assert_allclose(got[a + i], want[0], atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("window", [0, -1, -5])
def test_context_window_zero_or_negative_is_causal(window):
    # the extend kernel applies a window only when it is positive
    # (sglang.patch:527-541): 0 and negative values are plain causal
    # attention over the prefix, not "keys at the query's own position only"
    rng = np.random.default_rng(8)
    q, ke, ve, kp, vp, qo, kv, idx = _segments(rng, 4, 2, 8, [7, 3], [5, 0])
    kpos = np.arange(5)
    qpos = np.r_[np.arange(5, 12), np.arange(3)]
    base = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.5, q_positions=qpos, kv_positions=kpos)
    got = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.5, window=window, q_positions=qpos,
                               kv_positions=kpos)
    np.testing.assert_array_equal(got, base)
    # and a window of 1 does restrict (each query sees keys at q_pos - 1 .. q_pos)
    one = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.5, window=1, q_positions=qpos, kv_positions=kpos)
    assert not np.allclose(one, base)


def test_context_sinks_scale_by_sigmoid_of_lse():
    rng = np.random.default_rng(6)
    hq, hkv, d = 4, 1, 8
    q, ke, ve, kp, vp, qo, kv, idx = _segments(rng, hq, hkv, d, [6], [5])
    sinks = rng.standard_normal(hq).astype(np.float32)
    base = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.4)
    got = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, 0.4, sinks=sinks)
    keys = np.concatenate((kp[idx], ke)).astype(np.float64)
    for i in range(6):
        s = 0.4 * np.einsum("nd,hd->hn", keys[: 5 + i + 1, 0, :], q[i].astype(np.float64))
        lse = torch.logsumexp(torch.from_numpy(s), dim=1).numpy()
        want = base[i] * torch.sigmoid(torch.from_numpy(lse - sinks)).numpy()[:, None]
        np.testing.assert_allclose(got[i], want, atol=1e-6, rtol=1e-5)


def test_context_logit_cap_equals_sdpa_on_capped_keys():
    """A soft cap is a per-score transform.  With queries that read one key
    dimension only (q = a e0), each score is scale * a * k[0]; uncapped
    attention over keys whose first dim is replaced by
    cap * tanh(scale * a * k[0] / cap) / (scale * a) (numpy's tanh) has
    exactly the capped scores, so SDPA over those keys is the capped
    oracle's answer.  Scores spread over +-40 against caps of 5 and 30, so a
    cap on the unscaled score, a cap without the outer factor or none at all
    all fail."""
    rng = np.random.default_rng(12)
    hq = hkv = 2
    d = 8
    q_lens, p_lens = [6, 1, 9], [5, 0, 13]
    q, ke, ve, kp, vp, qo, kv, idx = _segments(rng, hq, hkv, d, q_lens, p_lens)
    amp = np.array([1.5, -2.0])
    q[:] = 0.0
    q[:, :, 0] = amp[None, :]
    ke[:, :, 0] = rng.uniform(-60, 60, size=ke.shape[:2])
    kp[:, :, 0] = rng.uniform(-60, 60, size=kp.shape[:2])
    scale = 0.45
    for cap in (5.0, 30.0):
        got = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, scale, logit_cap=cap)
        for s in range(len(q_lens)):
            a, b, x, y = qo[s], qo[s + 1], kv[s], kv[s + 1]
            n, plen = b - a, y - x
            keys = np.concatenate((kp[idx[x:y]], ke[a:b])).astype(np.float64)
            vals = np.concatenate((vp[idx[x:y]], ve[a:b])).astype(np.float64)
            mask = np.zeros((n, plen + n), dtype=bool)
            mask[:, :plen] = True
            mask[:, plen:] = np.tril(np.ones((n, n), dtype=bool))
            for h in range(hq):
                capped = keys.copy()
                sc = scale * amp[h] * keys[:, h, 0]
                capped[:, h, 0] = cap * np.tanh(sc / cap) / (scale * amp[h])
                want = _sdpa(q[a:b, h : h + 1], capped[:, h : h + 1], vals[:, h : h + 1], mask, scale)
                np.testing.assert_allclose(got[a:b, h : h + 1], want, atol=1e-6, rtol=1e-5)
        uncapped = at.context_attention(q, ke, ve, kp, vp, qo, kv, idx, scale)
        assert np.abs(got - uncapped).max() > 1e-2
