"""CPU restatement of one GQA decode step with attention sinks (fp32).

Semantics of the reference's sink normalisation
(``akv/system/sglang/srt/layers/attention/context_backend.py:254-272``):
the attention library returns the softmax output ``o`` and the natural-log
LSE of the scaled scores; the result is ``o * sigmoid(lse - sink)``, i.e.
``sum_j e^{s_j} v_j / (sum_j e^{s_j} + e^{sink})``.  Restated here directly
in the second form.

Pinned by (``tests/test_oracle_attention.py``): without sinks it equals
``torch.nn.functional.scaled_dot_product_attention`` in fp32; with sinks it
equals the reference's first form computed from ``torch.logsumexp``; one key
reduces to ``v e^s / (e^s + e^sink)``.

``context_attention`` (the prefill over context segments) is pinned against
causal SDPA (no prefix), SDPA with an explicit prefix-plus-causal mask, the
reference's own windowed gather (``native_plan``: ``searchsorted`` of
``q_pos - window`` over the segment's ordered key positions, then plain
attention per query, ``context_backend.py:196-238``), and the sink form;
its logit cap against SDPA over keys whose one score-carrying dimension
holds the capped score (queries that read only that dimension).
"""

import numpy as np


def decode_attention(q, keys, values, scale, sinks=None):
    """``q``: [Hq, D]; ``keys``/``values``: [N, Hkv, D]; returns [Hq, D] fp32."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    v = np.asarray(values, dtype=np.float64)
    hq = q.shape[0]
    hkv = k.shape[1] if k.ndim == 3 else 1
    group = hq // hkv
    out = np.zeros(q.shape, dtype=np.float64)
    for h in range(hq):
        g = h // group
        if len(k) == 0:
            continue
        s = scale * (k[:, g, :] @ q[h])
        m = s.max()
        if sinks is not None:
            m = max(m, float(sinks[h]))
        e = np.exp(s - m)
        denom = e.sum() + (np.exp(float(sinks[h]) - m) if sinks is not None else 0.0)
        out[h] = (e[:, None] * v[:, g, :]).sum(0) / denom
    return out.astype(np.float32)


def context_attention(q, k_ext, v_ext, k_pool, v_pool, qo_indptr, kv_indptr, kv_indices, scale, *,
                      window=-1, q_positions=None, kv_positions=None, sinks=None, logit_cap=0.0):
    """Prefill (extend) attention of context segments, in float64.

    Restates the extend attention with context positions
    (``akv/system/sglang/srt/layers/attention/context_backend.py:180-251``,
    ``akv/system/sglang.patch:106-237``): segment ``s`` has queries
    ``qo_indptr[s]..qo_indptr[s+1]`` and prefix keys
    ``kv_indices[kv_indptr[s]..kv_indptr[s+1]]`` (pool rows, all visible),
    then its own keys ``k_ext``/``v_ext`` causally (key ``j <= i``).  With
    ``window > 0`` a key is visible only when ``q_pos <= k_pos + window``
    (the extend kernel applies no window for 0 or less,
    ``akv/system/sglang.patch:527-541``); without positions
    ``q_pos = prefix_length + i`` and prefix ``k_pos = j``.  With
    ``logit_cap > 0`` every scaled score ``s`` becomes
    ``logit_cap * tanh(s / logit_cap)`` before the softmax; sinks are not
    capped.  The cap is applied inside SGLang's extend-attention Triton
    kernel (``sglang==0.5.20+akv``, upstream base commit 94602c9c,
    ``akv/system/pyproject.toml:13,32``; not part of the reference tree),
    which scales the score first and caps it second; the reference passes
    the layer's cap to it at ``akv/system/sglang.patch:2437,2459``.

    ``q``: [Nq, Hq, D]; ``k_ext``/``v_ext``: [Nq, Hkv, D]; ``k_pool``/``v_pool``:
    [slots, Hkv, D].  Returns [Nq, Hq, D] float32.
    """
    q = np.asarray(q, dtype=np.float64)
    ke = np.asarray(k_ext, dtype=np.float64)
    ve = np.asarray(v_ext, dtype=np.float64)
    kp = np.asarray(k_pool, dtype=np.float64)
    vp = np.asarray(v_pool, dtype=np.float64)
    qo = np.asarray(qo_indptr, dtype=np.int64)
    kv = np.asarray(kv_indptr, dtype=np.int64)
    idx = np.asarray(kv_indices, dtype=np.int64)
    hq, hkv = q.shape[1], ke.shape[1]
    group = hq // hkv
    out = np.zeros(q.shape, dtype=np.float64)
    for s in range(len(qo) - 1):
        a, b = qo[s], qo[s + 1]
        x, y = kv[s], kv[s + 1]
        plen = y - x
        slots = idx[x:y]
        if q_positions is None:
            qpos = plen + np.arange(b - a)
            kpos = np.arange(plen)
        else:
            qpos = np.asarray(q_positions, dtype=np.int64)[a:b]
            kpos = np.asarray(kv_positions, dtype=np.int64)[x:y]
        keys_k = np.concatenate((kp[slots], ke[a:b]), 0)  # [plen + n, Hkv, D]
        keys_v = np.concatenate((vp[slots], ve[a:b]), 0)
        keys_pos = np.concatenate((kpos, qpos))
        for i in range(b - a):
            vis = np.zeros(plen + b - a, dtype=bool)
            vis[:plen] = True
            vis[plen : plen + i + 1] = True
            if window > 0:
                vis &= qpos[i] <= keys_pos + window
            for h in range(hq):
                g = h // group
                sc = scale * (keys_k[vis, g, :] @ q[a + i, h])
                if logit_cap > 0:
                    sc = logit_cap * np.tanh(sc / logit_cap)
                m = sc.max() if len(sc) else -np.inf
                if sinks is not None:
                    m = max(m, float(sinks[h]))
                e = np.exp(sc - m)
                den = e.sum() + (np.exp(float(sinks[h]) - m) if sinks is not None else 0.0)
                out[a + i, h] = (e[:, None] * keys_v[vis, g, :]).sum(0) / den if den > 0 else 0.0
    return out.astype(np.float32)
