"""GPU parity of the prefill context attention (MFMA) against the float64
oracle: ragged segments, empty and long prefixes, GQA groups 8 and 4 and
groups that are not powers of two, head dims 64 and 128 and narrower ones
(multiples of 8), logit caps, position-based sliding windows over positions
with holes, the native (position-free) window, sinks, bf16 and f32 outputs;
and batch metadata of plain requests bound to physical slots."""

import numpy as np
import pytest
import torch

from akv_amd import context_attention as ca
from oracle import attention as oat

from harness import attention_metadata, plain_segments, prefill_forward

pytestmark = pytest.mark.gpu

TOL = 2e-2  # abs, bf16 inputs and P in bf16 (the decode check's tolerance)


def _f32(t):
    return t.detach().float().cpu().numpy()


def _case(device, hq, hkv, d, q_lens, p_lens, seed, slots=4000):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    nq = sum(q_lens)
    q = torch.randn((nq, hq, d), generator=g).to(torch.bfloat16)
    ke = torch.randn((nq, hkv, d), generator=g).to(torch.bfloat16)
    ve = torch.randn((nq, hkv, d), generator=g).to(torch.bfloat16)
    kp = torch.randn((slots, hkv, d), generator=g).to(torch.bfloat16)
    vp = torch.randn((slots, hkv, d), generator=g).to(torch.bfloat16)
    qo = np.concatenate(([0], np.cumsum(q_lens))).astype(np.int64)
    kv = np.concatenate(([0], np.cumsum(p_lens))).astype(np.int64)
    idx = rng.integers(1, slots, size=kv[-1]).astype(np.int32)
    # ordered positions with holes: prefix first, then the queries
    kpos, qpos = [], []
    for n, p in zip(q_lens, p_lens):
        allp = np.sort(rng.choice(4 * (n + p) + 8, size=n + p, replace=False))
        kpos.append(allp[:p])
        qpos.append(allp[p:])
    kpos = np.concatenate(kpos).astype(np.int64)
    qpos = np.concatenate(qpos).astype(np.int64)
    dev = {k: v.to(device) for k, v in dict(q=q, ke=ke, ve=ve, kp=kp, vp=vp).items()}
    return dict(q=q, ke=ke, ve=ve, kp=kp, vp=vp, qo=qo, kv=kv, idx=idx, kpos=kpos, qpos=qpos, dev=dev)


def _run(device, c, *, window, positions, sinks, out_dtype, scale, logit_cap=0.0):
    dv = c["dev"]
    out = torch.full(dv["q"].shape, 7.0, dtype=out_dtype, device=device)
    qo = torch.from_numpy(c["qo"]).to(device)
    kv = torch.from_numpy(c["kv"]).to(device)
    idx = torch.from_numpy(c["idx"]).to(device)
    qp = torch.from_numpy(c["qpos"]).to(device) if positions else None
    kp = torch.from_numpy(c["kpos"]).to(device) if positions else None
    ca.extend_attention_fwd(dv["q"], dv["ke"], dv["ve"], out, dv["kp"], dv["vp"], qo, kv, idx, None, True, None,
                            int(np.diff(c["qo"]).max()), sm_scale=scale, logit_cap=logit_cap,
                            sliding_window_size=window, sinks=sinks, context_q_positions=qp, context_kv_positions=kp)
    torch.cuda.synchronize()
    want = oat.context_attention(_f32(c["q"]), _f32(c["ke"]), _f32(c["ve"]), _f32(c["kp"]), _f32(c["vp"]),
                                 c["qo"], c["kv"], c["idx"], scale, window=window,
                                 q_positions=c["qpos"] if positions else None,
                                 kv_positions=c["kpos"] if positions else None,
                                 sinks=_f32(sinks) if sinks is not None else None, logit_cap=logit_cap)
    return _f32(out), want


# groups that are not powers of two (padded rows), heads narrower than the
# 64- / 128-dim tiles, logit caps, alone and together, with windows and sinks
@pytest.mark.parametrize("d,hq,hkv,cap", [
    (128, 28, 4, 0.0), (64, 12, 4, 0.0), (64, 40, 8, 0.0), (128, 7, 7, 0.0),
    (80, 8, 8, 0.0), (96, 16, 2, 0.0), (32, 8, 1, 0.0), (112, 6, 2, 0.0), (8, 4, 4, 0.0),
    (64, 64, 8, 30.0), (128, 32, 8, 5.0), (96, 24, 8, 20.0), (64, 6, 1, 2.0),
])
@pytest.mark.parametrize("window,positions,with_sinks", [(-1, False, False), (24, True, True)])
def test_groups_head_dims_and_caps(device, d, hq, hkv, cap, window, positions, with_sinks):
    c = _case(device, hq, hkv, d, Q_LENS, P_LENS, seed=3 * d + hq + int(cap) + window)
    sinks = (torch.randn(hq, generator=torch.Generator().manual_seed(2)) * 2).to(device) if with_sinks else None
    print(f"context attention d={d} hq={hq} hkv={hkv} cap={cap} window={window} sinks={with_sinks}", flush=True)
    got, want = _run(device, c, window=window, positions=positions, sinks=sinks, out_dtype=torch.float32,
                     scale=d ** -0.5, logit_cap=cap)
    for s in range(len(Q_LENS)):
        a, b = c["qo"][s], c["qo"][s + 1]
        err = np.abs(got[a:b] - want[a:b]).max()
        assert err <= TOL, f"segment {s} (q {Q_LENS[s]}, prefix {P_LENS[s]}) max err {err}"


def test_capped_scores_far_apart(device):
    """Capped logits with the scores spread ~50x the cap: the softmax sees
    values in [-cap, cap] only, whatever Q and K hold."""
    c = _case(device, 16, 4, 64, [70, 300], [500, 40], seed=77)
    c["q"] = c["q"] * 8
    c["dev"]["q"] = c["q"].to(device)
    got, want = _run(device, c, window=-1, positions=False, sinks=None, out_dtype=torch.float32, scale=0.125,
                     logit_cap=3.0)
    assert np.abs(got - want).max() <= TOL


Q_LENS = [1, 15, 16, 17, 100, 300, 5]
P_LENS = [0, 5, 64, 1000, 0, 37, 130]


@pytest.mark.parametrize("d,hq,hkv", [(64, 64, 8), (128, 32, 8)])
# window 0 is no window, as in the extend kernel the prefill replaces
@pytest.mark.parametrize("window,positions", [(-1, False), (24, True), (24, False), (0, True)])
@pytest.mark.parametrize("with_sinks", [True, False])
def test_segments_match_oracle(device, d, hq, hkv, window, positions, with_sinks):
    c = _case(device, hq, hkv, d, Q_LENS, P_LENS, seed=d + hq + window + with_sinks)
    sinks = (torch.randn(hq, generator=torch.Generator().manual_seed(1)) * 2).to(device) if with_sinks else None
    print(f"context attention d={d} hq={hq} window={window} positions={positions} sinks={with_sinks}", flush=True)
    for out_dtype in (torch.bfloat16, torch.float32):
        got, want = _run(device, c, window=window, positions=positions, sinks=sinks, out_dtype=out_dtype,
                         scale=d ** -0.5)
        for s in range(len(Q_LENS)):
            a, b = c["qo"][s], c["qo"][s + 1]
            err = np.abs(got[a:b] - want[a:b]).max()
            assert err <= TOL, f"segment {s} (q {Q_LENS[s]}, prefix {P_LENS[s]}) max err {err}"


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("idx_dtype,pos_dtype,indptr_dtype", [(torch.int64, torch.int32, torch.int32),
                                                              (torch.int32, torch.int32, torch.int64)])
def test_index_dtypes(device, idx_dtype, pos_dtype, indptr_dtype, d):
    """int32 / int64 indices, positions and indptrs take their own kernel paths."""
    hq, hkv = 16, 2
    c = _case(device, hq, hkv, d, [33, 70], [100, 9], seed=31)
    dv = c["dev"]
    qo = torch.from_numpy(c["qo"]).to(indptr_dtype).to(device)
    kv = torch.from_numpy(c["kv"]).to(indptr_dtype).to(device)
    idx = torch.from_numpy(c["idx"]).to(idx_dtype).to(device)
    qp = torch.from_numpy(c["qpos"]).to(pos_dtype).to(device)
    kp = torch.from_numpy(c["kpos"]).to(pos_dtype).to(device)
    out = torch.empty(dv["q"].shape, dtype=torch.float32, device=device)
    ca.extend_attention_fwd(dv["q"], dv["ke"], dv["ve"], out, dv["kp"], dv["vp"], qo, kv, idx, None, True, None, 70,
                            sm_scale=0.125, sliding_window_size=16, context_q_positions=qp, context_kv_positions=kp)
    torch.cuda.synchronize()
    want = oat.context_attention(_f32(c["q"]), _f32(c["ke"]), _f32(c["ve"]), _f32(c["kp"]), _f32(c["vp"]),
                                 c["qo"], c["kv"], c["idx"], 0.125, window=16, q_positions=c["qpos"],
                                 kv_positions=c["kpos"])
    assert np.abs(_f32(out) - want).max() <= TOL


@pytest.mark.parametrize("d,idx_dtype", [(64, torch.int32), (128, torch.int64)])
def test_strided_pool_and_extend_views(device, d, idx_dtype):
    """K/V pools and extend rows that are views into wider buffers (slot and
    token strides beyond one row): the tile loads address rows by stride."""
    hq, hkv, extra = 16, 2, 3
    c = _case(device, hq, hkv, d, [40, 17], [130, 64], seed=5)
    g = torch.Generator().manual_seed(6)
    dv = c["dev"]

    def widen(t):
        big = torch.randn((t.shape[0], t.shape[1] + extra, d), generator=g).to(torch.bfloat16).to(device)
        big[:, 1 : 1 + t.shape[1]] = t
        return big[:, 1 : 1 + t.shape[1]]

    kp, vp, ke, ve = widen(dv["kp"]), widen(dv["vp"]), widen(dv["ke"]), widen(dv["ve"])
    assert not kp.is_contiguous() and kp.stride(0) == (hkv + extra) * d
    qo = torch.from_numpy(c["qo"]).to(device)
    kv = torch.from_numpy(c["kv"]).to(device)
    idx = torch.from_numpy(c["idx"]).to(idx_dtype).to(device)
    out = torch.empty(dv["q"].shape, dtype=torch.float32, device=device)
    ca.extend_attention_fwd(dv["q"], ke, ve, out, kp, vp, qo, kv, idx, None, True, None, 40, sm_scale=d ** -0.5,
                            sliding_window_size=-1)
    torch.cuda.synchronize()
    want = oat.context_attention(_f32(c["q"]), _f32(c["ke"]), _f32(c["ve"]), _f32(c["kp"]), _f32(c["vp"]),
                                 c["qo"], c["kv"], c["idx"], d ** -0.5)
    assert np.abs(_f32(out) - want).max() <= TOL


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (32, 2), (64, 2), (6, 3), (8, 1)])
def test_group_sizes(device, d, hq, hkv):
    """GQA groups of 1, 2, 16 and 32 q heads per KV head, and 3 or 1 KV heads
    (the grid's KV head is the workgroup id modulo their count): a block
    holds rows_per_block / group tokens (512 down to 8), with causal, prefix,
    window and sink handling unchanged."""
    c = _case(device, hq, hkv, d, [3, 70, 300], [0, 45, 200], seed=hq + d)
    sinks = (torch.randn(hq, generator=torch.Generator().manual_seed(3))).to(device)
    got, want = _run(device, c, window=32, positions=True, sinks=sinks, out_dtype=torch.float32, scale=d ** -0.5)
    assert np.abs(got - want).max() <= TOL
    got, want = _run(device, c, window=-1, positions=False, sinks=None, out_dtype=torch.bfloat16, scale=d ** -0.5)
    assert np.abs(got - want).max() <= TOL


def test_metadata_from_plain_requests(device):
    """Batch metadata of plain requests (prefix, then queries) bound to
    permuted physical slots -> one launch."""
    hq, hkv, d = 64, 8, 64
    requests = [plain_segments(37, 20), plain_segments(0, 70), plain_segments(300, 1)]
    n_occ = sum(r.occurrences for r in requests)
    rng = np.random.default_rng(0)
    slots = torch.from_numpy(rng.permutation(np.arange(1, 1 + n_occ)).astype(np.int64)).to(device)
    meta = attention_metadata(requests, slots)
    g = torch.Generator().manual_seed(2)
    nq = meta.query_count
    q = torch.randn((nq, hq, d), generator=g).to(torch.bfloat16).to(device)
    ke = torch.randn((nq, hkv, d), generator=g).to(torch.bfloat16).to(device)
    ve = torch.randn((nq, hkv, d), generator=g).to(torch.bfloat16).to(device)
    pool_k = torch.randn((n_occ + 1, hkv, d), generator=g).to(torch.bfloat16).to(device)
    pool_v = torch.randn((n_occ + 1, hkv, d), generator=g).to(torch.bfloat16).to(device)
    out = torch.empty_like(q)
    prefill_forward(meta, q, ke, ve, out, pool_k, pool_v, sliding_window_size=-1)
    torch.cuda.synchronize()
    c = meta.cpu
    want = oat.context_attention(_f32(q), _f32(ke), _f32(ve), _f32(pool_k), _f32(pool_v), c.qo_indptr, c.kv_indptr,
                                 slots.cpu().numpy()[c.occurrences], d ** -0.5, q_positions=c.query_positions,
                                 kv_positions=c.kv_positions)
    assert np.abs(_f32(out) - want).max() <= TOL


LEVEL_PROFILES = {
    # log2-domain score level of prefix tile t (64 keys) above tile 0
    "ramp": lambda t: 25.0 * t,  # each tile 25 above the last: sums pass 2^32 every other tile
    "jump40": lambda t: 40.0 * (t > 0),  # one tile's sum near 2^46: renormalised
    "jump70": lambda t: 70.0 * (t > 0),  # near 2^76, past 2^64: the workgroup restarts exactly
    "jump300": lambda t: 300.0 * (t > 0),  # 2^300 overflows to inf: restart
    "drop": lambda t: -200.0 * (t > 0),  # later keys underflow to zero weight
}


@pytest.mark.parametrize("d,hq,hkv", [(64, 64, 8), (128, 32, 8)])
@pytest.mark.parametrize("profile", sorted(LEVEL_PROFILES))
@pytest.mark.parametrize("window", [-1, 100])
def test_score_levels_across_tiles(device, d, hq, hkv, profile, window):
    """Prefix keys whose scores sit far above (or below) the first tile's:
    the running maximum comes from the first tile's exact row maxima, later
    tiles skip the maxima, and their weight sums decide between keeping it,
    renormalising by a power of two, and restarting the keys with exact
    maxima.  Every case matches the float64 oracle, sinks included."""
    scale = d ** -0.5
    c = scale * 1.4426950408889634  # log2-domain scale
    q_lens, p_lens, slots = [40, 200], [64 * 6, 64 * 3 + 10], 1200
    g = torch.Generator().manual_seed(7 + d)
    rng = np.random.default_rng(d)
    nq = sum(q_lens)
    q = torch.randn((nq, hq, d), generator=g) * 0.5
    q[..., 0] = 8.0
    ke = (torch.randn((nq, hkv, d), generator=g) * 0.5).to(torch.bfloat16)
    ve = torch.randn((nq, hkv, d), generator=g).to(torch.bfloat16)
    kp = torch.randn((slots, hkv, d), generator=g) * 0.5
    vp = torch.randn((slots, hkv, d), generator=g).to(torch.bfloat16)
    qo = np.concatenate(([0], np.cumsum(q_lens))).astype(np.int64)
    kv = np.concatenate(([0], np.cumsum(p_lens))).astype(np.int64)
    idx = (rng.permutation(slots - 1)[: kv[-1]] + 1).astype(np.int32)  # distinct slots
    level = LEVEL_PROFILES[profile]
    for s in range(len(p_lens)):
        for j in range(p_lens[s]):
            kp[idx[kv[s] + j], :, 0] = level(j // 64) / (c * 8.0)
    q, kp = q.to(torch.bfloat16), kp.to(torch.bfloat16)
    positions = window >= 0
    kpos = np.concatenate([np.arange(p) * 2 for p in p_lens]).astype(np.int64)
    qpos = np.concatenate([2 * p + np.arange(n) for n, p in zip(q_lens, p_lens)]).astype(np.int64)
    sinks = torch.randn(hq, generator=torch.Generator().manual_seed(11)).to(device)
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device=device)
    dq, dke, dve, dkp, dvp = (t.to(device) for t in (q, ke, ve, kp, vp))
    print(f"score levels d={d} profile={profile} window={window}", flush=True)
    ca.extend_attention_fwd(dq, dke, dve, out, dkp, dvp, torch.from_numpy(qo).to(device),
                            torch.from_numpy(kv).to(device), torch.from_numpy(idx).to(device), None, True, None,
                            max(q_lens), sm_scale=scale, sliding_window_size=window, sinks=sinks,
                            context_q_positions=torch.from_numpy(qpos).to(device) if positions else None,
                            context_kv_positions=torch.from_numpy(kpos).to(device) if positions else None)
    torch.cuda.synchronize()
    want = oat.context_attention(_f32(q), _f32(ke), _f32(ve), _f32(kp), _f32(vp), qo, kv, idx, scale,
                                 window=window, q_positions=qpos if positions else None,
                                 kv_positions=kpos if positions else None, sinks=_f32(sinks))
    got = _f32(out)
    assert np.isfinite(got).all()
    assert np.abs(got - want).max() <= TOL


@pytest.mark.parametrize("mag", [1.0, 3.0])
@pytest.mark.parametrize("seed", range(10))
def test_random_layouts(device, seed, mag):
    """Seeded random batches: 1-4 segments of 1-299 queries over 0-699
    prefix keys, head_dim 64 or 128, 1-8 KV heads, groups of 1-16, windows
    none / 0 / 7 / 64 / 200 with and without positions, with and without
    sinks; Q and K scaled by ``mag`` (3 puts the scores' spread near 40 in
    the log2 domain, where a bf16 rounding of the scaled Q would already
    cost several times the tolerance)."""
    rng = np.random.default_rng(1000 + seed)
    d = [64, 128][seed % 2]
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 4, 8, 16]))
    n_seg = int(rng.integers(1, 5))
    q_lens = rng.integers(1, 300, n_seg)
    p_lens = rng.integers(0, 700, n_seg)
    window = int(rng.choice([-1, -1, 0, 7, 64, 200]))
    positions = bool(rng.random() < 0.5)
    with_sinks = bool(rng.random() < 0.5)
    slots = int(p_lens.sum()) + 16
    g = torch.Generator().manual_seed(seed)
    nq = int(q_lens.sum())
    q = (torch.randn((nq, hq, d), generator=g) * mag).to(torch.bfloat16)
    ke = (torch.randn((nq, hkv, d), generator=g) * mag).to(torch.bfloat16)
    ve = torch.randn((nq, hkv, d), generator=g).to(torch.bfloat16)
    kp = (torch.randn((slots, hkv, d), generator=g) * mag).to(torch.bfloat16)
    vp = torch.randn((slots, hkv, d), generator=g).to(torch.bfloat16)
    qo = np.concatenate(([0], np.cumsum(q_lens))).astype(np.int64)
    kv = np.concatenate(([0], np.cumsum(p_lens))).astype(np.int64)
    idx = (rng.permutation(slots - 1)[: kv[-1]] + 1).astype(np.int32)
    kpos, qpos = [], []
    for n, p in zip(q_lens, p_lens):
        allp = np.sort(rng.choice(3 * (n + p) + 8, size=n + p, replace=False))
        kpos.append(allp[:p])
        qpos.append(allp[p:])
    kpos = np.concatenate(kpos).astype(np.int64)
    qpos = np.concatenate(qpos).astype(np.int64)
    sinks = (torch.randn(hq, generator=g) * 2).to(device) if with_sinks else None
    scale = d ** -0.5
    print(f"random layout seed={seed} mag={mag} d={d} hq={hq} hkv={hkv} segments={n_seg} window={window} "
          f"positions={positions} sinks={with_sinks}", flush=True)
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device=device)
    ca.extend_attention_fwd(q.to(device), ke.to(device), ve.to(device), out, kp.to(device), vp.to(device),
                            torch.from_numpy(qo).to(device), torch.from_numpy(kv).to(device),
                            torch.from_numpy(idx).to(device), None, True, None, int(q_lens.max()),
                            sm_scale=scale, sliding_window_size=window, sinks=sinks,
                            context_q_positions=torch.from_numpy(qpos).to(device) if positions else None,
                            context_kv_positions=torch.from_numpy(kpos).to(device) if positions else None)
    torch.cuda.synchronize()
    want = oat.context_attention(_f32(q), _f32(ke), _f32(ve), _f32(kp), _f32(vp), qo, kv, idx, scale,
                                 window=window, q_positions=qpos if positions else None,
                                 kv_positions=kpos if positions else None,
                                 sinks=_f32(sinks) if sinks is not None else None)
    assert np.abs(_f32(out) - want).max() <= TOL


def test_rejects_nonpositive_scale(device):
    """Masked scores are -inf before scaling, so the scale must be positive."""
    c = _case(device, 16, 2, 64, [5], [3], seed=4)
    dv = c["dev"]
    out = torch.empty(dv["q"].shape, dtype=torch.float32, device=device)
    qo = torch.from_numpy(c["qo"]).to(device)
    kv = torch.from_numpy(c["kv"]).to(device)
    idx = torch.from_numpy(c["idx"]).to(device)
    for scale in (0.0, -0.125, float("nan")):
        with pytest.raises(ValueError, match="scale must be positive"):
            ca.extend_attention_fwd(dv["q"], dv["ke"], dv["ve"], out, dv["kp"], dv["vp"], qo, kv, idx, None, True,
                                    None, 5, sm_scale=scale)
