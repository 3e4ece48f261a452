"""The allocation-free decode attention entry point against the ordinary one.

akv_decode_attention_noalloc keeps its split-K partials in a static device
array instead of a caller workspace; everything else is the same kernels.
Two calls in a row (the second smaller) must match akv_decode_attention bit
for bit, and a call whose partials exceed the array is rejected before any
launch.
"""

import numpy as np
import pytest
import torch

from akv_amd import _lib, attention
from akv_amd.ops import current_stream_handle

pytestmark = pytest.mark.gpu


def _case(device, seed, n_requests, q_heads, kv_heads, head_dim, max_keys, slots=4096):
    g = torch.Generator(device="cpu").manual_seed(seed)
    rng = np.random.default_rng(seed)
    lengths = rng.integers(0, max_keys + 1, size=n_requests)
    lengths[0] = max_keys
    indptr = np.zeros(n_requests + 1, dtype=np.int32)
    indptr[1:] = np.cumsum(lengths)
    indices = rng.integers(1, slots, size=int(indptr[-1])).astype(np.int32)
    mk = lambda *shape: torch.randn(shape, generator=g).to(torch.bfloat16).to(device)  # noqa: E731
    return dict(
        q=mk(n_requests, q_heads, head_dim), k=mk(slots, kv_heads, head_dim), v=mk(slots, kv_heads, head_dim),
        indptr=torch.from_numpy(indptr).to(device), indices=torch.from_numpy(indices).to(device),
        sinks=torch.randn(q_heads, generator=g).to(device), max_len=int(max_keys),
    )


def _noalloc(c, out, scale):
    lib = _lib.load()
    q, k, v = c["q"], c["k"], c["v"]
    n, hq, d = q.shape
    rc = lib.akv_decode_attention_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0),
        v.stride(1), n, hq, k.shape[1], d, c["indptr"].data_ptr(), c["indices"].data_ptr(), c["sinks"].data_ptr(),
        scale, out.data_ptr(), _lib.AKV_F32 if out.dtype == torch.float32 else _lib.AKV_BF16, out.stride(0),
        out.stride(1), c["max_len"], None, current_stream_handle(q.device))
    _lib.check(rc, "akv_decode_attention_noalloc")


@pytest.mark.parametrize("head_dim,out_dtype", [(64, torch.bfloat16), (128, torch.float32)])
def test_noalloc_matches_workspace_entry_twice(device, head_dim, out_dtype):
    scale = head_dim ** -0.5
    for call, (n, keys, seed) in enumerate([(6, 3000, 1), (3, 700, 2)]):
        c = _case(device, seed + head_dim, n, 16, 2, head_dim, keys)
        print(f"noalloc decode attention: call {call}, d={head_dim}, {n} requests, max {keys} keys", flush=True)
        want = torch.empty(c["q"].shape, dtype=out_dtype, device=device)
        attention.decode_attention(c["q"], c["k"], c["v"], c["indptr"], c["indices"], want, scale=scale,
                                   max_len=c["max_len"], sinks=c["sinks"])
        got = torch.full(c["q"].shape, float("nan"), dtype=out_dtype, device=device)
        _noalloc(c, got, scale)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {call}: max diff {(got.float() - want.float()).abs().max()}"


def test_noalloc_rejects_more_than_the_static_scratch(device):
    lib = _lib.load()
    limit = lib.akv_decode_attention_noalloc_max_bytes()
    assert limit == 32 << 20
    c = _case(device, 5, 2, 8, 1, 64, 10)
    need_len = 10 ** 7  # 2 requests x 1 KV head x 39063 chunks x 16 x 66 floats > 32 MiB
    assert lib.akv_decode_attention_workspace_bytes(2, 1, 64, need_len) > limit
    out = torch.empty(c["q"].shape, dtype=torch.bfloat16, device=device)
    c["max_len"] = need_len
    with pytest.raises(ValueError, match="static scratch holds"):
        _noalloc(c, out, 0.125)
