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
