"""GPU parity of the decode-attention consumer (MFMA) and the end-to-end
decode check over Drop + Reposition metadata (GPT-OSS decode shape)."""


import numpy as np
import pytest
import torch

from akv_amd import attention, ops, synth, tables
from oracle import attention as oat
from oracle import occurrence as occ

from harness import window_indices

pytestmark = pytest.mark.gpu

TOL = 2e-2  # abs, bf16 outputs (the decode check's tolerance)


def _f32(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("with_sinks", [True, False])
# mag scales Q and K: 3 spreads the scores over ~40 in the log2 domain
@pytest.mark.parametrize("mag", [1.0, 3.0])
# long: split over key chunks, merged by the combine; short (at most one
# 256-key chunk): normalised by the one launch
@pytest.mark.parametrize("lengths", [[0, 1, 15, 16, 17, 255, 256, 257, 1000, 5000],
                                     [0, 1, 15, 16, 17, 100, 129, 255, 256]], ids=["long", "short"])
def test_random_lengths_match_oracle(device, head_dim, with_sinks, mag, lengths):
    g = torch.Generator().manual_seed(head_dim + with_sinks)
    rng = np.random.default_rng(head_dim)
    slots, hq, hkv = 20000, 64, 8
    k = (torch.randn((slots, hkv, head_dim), generator=g) * mag).to(torch.bfloat16).to(device)
    v = torch.randn((slots, hkv, head_dim), generator=g).to(torch.bfloat16).to(device)
    indptr = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    idx = rng.integers(1, slots, size=indptr[-1]).astype(np.int32)
    q = (torch.randn((len(lengths), hq, head_dim), generator=g) * mag).to(torch.bfloat16).to(device)
    sinks = (torch.randn(hq, generator=g) * 2).to(device) if with_sinks else None
    scale = head_dim ** -0.5
    for out_dtype in (torch.bfloat16, torch.float32):
        out = torch.full((len(lengths), hq, head_dim), 7.0, dtype=out_dtype, device=device)
        attention.decode_attention(q, k, v, torch.from_numpy(indptr).to(device), torch.from_numpy(idx).to(device),
                                   out, scale=scale, max_len=max(lengths), sinks=sinks)
        torch.cuda.synchronize()
        got = _f32(out)
        kk, vv, qq = _f32(k), _f32(v), _f32(q)
        s_np = _f32(sinks) if sinks is not None else None
        for b, n in enumerate(lengths):
            sel = idx[indptr[b] : indptr[b + 1]]
            want = oat.decode_attention(qq[b], kk[sel], vv[sel], scale, s_np)
            err = np.abs(got[b] - want).max()
            assert err <= TOL, f"request {b} (len {n}) max err {err}"


@pytest.mark.parametrize("seed", range(12))
def test_random_batches_match_oracle(device, seed):
    # seeded random batches: batch size, KV heads, GQA group (1-16), head
    # dim, ragged lengths (empty, inside one chunk, over many), a host bound
    # above the longest request (empty trailing chunks), sinks, spread and
    # output dtype all vary
    rng = np.random.default_rng(700 + seed)
    g = torch.Generator().manual_seed(700 + seed)
    head_dim = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 4, 8, 16]))
    B = int(rng.integers(1, 41))
    kind = rng.integers(0, 3, size=B)
    lengths = np.where(kind == 0, rng.integers(0, 3, size=B),
                       np.where(kind == 1, rng.integers(1, 257, size=B), rng.integers(257, 4001, size=B)))
    max_len = int(lengths.max()) + int(rng.choice([0, 0, 1, 300]))
    mag = float(rng.choice([1.0, 3.0]))
    slots = 12000
    print(f"decode random {seed}: B={B} hq={hq} hkv={hkv} d={head_dim} max_len={max_len} mag={mag}", flush=True)
    k = (torch.randn((slots, hkv, head_dim), generator=g) * mag).to(torch.bfloat16).to(device)
    v = torch.randn((slots, hkv, head_dim), generator=g).to(torch.bfloat16).to(device)
    indptr = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    idx = rng.integers(0, slots, size=indptr[-1]).astype(np.int32)
    q = (torch.randn((B, hq, head_dim), generator=g) * mag).to(torch.bfloat16).to(device)
    sinks = (torch.randn(hq, generator=g) * 2).to(device) if rng.random() < 0.5 else None
    out_dtype = torch.float32 if rng.random() < 0.5 else torch.bfloat16
    out = torch.full((B, hq, head_dim), 7.0, dtype=out_dtype, device=device)
    scale = head_dim ** -0.5
    attention.decode_attention(q, k, v, torch.from_numpy(indptr).to(device), torch.from_numpy(idx).to(device),
                               out, scale=scale, max_len=max_len, sinks=sinks)
    torch.cuda.synchronize()
    got, kk, vv, qq = _f32(out), _f32(k), _f32(v), _f32(q)
    s_np = _f32(sinks) if sinks is not None else None
    for b, n in enumerate(lengths):
        sel = idx[indptr[b] : indptr[b + 1]]
        want = oat.decode_attention(qq[b], kk[sel], vv[sel], scale, s_np)
        err = np.abs(got[b] - want).max()
        assert err <= TOL, f"request {b} (len {n}) max err {err}"


def test_gpt_oss_decode_after_drop_and_reposition(device):
    """32 requests x 32k tokens: compaction -> Reposition of all 36 layers ->
    full / 128-window metadata -> one decode step on every layer (GPT-OSS
    alternates them: even layers sliding-window, odd layers full), each
    checked against the oracle on four requests."""
    w = synth.workload("gpt-oss-decode-32x32k")
    model = w.model
    assert model.n_layers == 36
    layouts = synth.compile_layouts(w)
    slots = synth.assign_slots(w, layouts)
    B, n = w.n_requests, w.lengths[0]
    # the generated token of each request sits in a slot no prompt token owns
    used = np.concatenate(slots.birth_rows + slots.fresh)
    gen_slot = np.setdiff1d(np.arange(1, w.pool_slots), used)[:B].astype(np.int32)
    table = torch.full((B, n + 4), -1, dtype=torch.int32)
    for b in range(B):
        table[b, n] = int(gen_slot[b])
    table = table.to(device)
    birth = torch.from_numpy(np.concatenate(slots.birth_rows)).to(device)
    fresh = torch.from_numpy(np.concatenate(slots.fresh)).to(device)
    inputs = tables.pack_compaction_inputs(layouts, device)
    out = tables.allocate_outputs(inputs, device, generated_total=B)
    rows = torch.arange(B, dtype=torch.int64, device=device)
    tables.compact_rows(inputs, table, rows, fresh, out, generated=torch.ones(B, dtype=torch.int32, device=device),
                        birth_slots=birth)
    pool = synth.make_pool(model, w.pool_slots, device, seed=9, generate_on_device=True)
    rope = synth.rope_table(w, device)
    # the lists feed the Reposition on the device, gated by the status word
    ops.reposition_kv_layers_gated(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src, out.copy_dst,
                                   out.copy_pairs, rope, status=out.status)

    # registry rows straight from the compaction outputs
    kept_off = np.concatenate(([0], np.cumsum(inputs.kept)))
    registry = torch.tensor(
        [(out.raw_indices.data_ptr() + 4 * int(kept_off[b]), out.active_positions.data_ptr() + 4 * int(kept_off[b]),
          n, inputs.kept[b], layouts[b].next_position, 0) for b in range(B)], dtype=torch.int64).to(device)
    seq = torch.tensor([k + 1 for k in inputs.kept], dtype=torch.int64, device=device)
    window = 128
    win_indptr = torch.zeros(B + 1, dtype=torch.int32, device=device)
    win_idx = torch.zeros(B * (window + 1), dtype=torch.int32, device=device)
    window_indices(registry, table, rows, seq, window, win_indptr, win_idx, status=out.status)

    g = torch.Generator().manual_seed(5)
    q = torch.randn((B, 64, 64), generator=g).to(torch.bfloat16).to(device)
    sinks = [torch.randn(64, generator=g).to(device) for _ in range(model.n_layers)]
    outs = []
    for layer in range(model.n_layers):
        ip, ix, mx = ((win_indptr, win_idx, window + 1) if layer % 2 == 0 else
                      (out.kv_indptr, out.kv_indices, max(inputs.kept) + 1))
        o = torch.empty((B, 64, 64), dtype=torch.bfloat16, device=device)
        attention.decode_attention(q, pool.k[layer], pool.v[layer], ip, ix, o, scale=0.125, max_len=mx,
                                   sinks=sinks[layer], status=out.status)
        outs.append(o)
    torch.cuda.synchronize()
    assert tables.check_status(out) == 0

    win_ip, win_ix = win_indptr.cpu().numpy(), win_idx.cpu().numpy()
    full_ip, full_ix = out.kv_indptr.cpu().numpy(), out.kv_indices.cpu().numpy()
    qq = _f32(q)
    for b in (0, 7, 19, 31):
        lay = layouts[b]
        cf = occ.closed_form(slots.birth_rows[b], lay.keep_mask.numpy(), lay.birth_positions.numpy(),
                             lay.positions.numpy(), slots.fresh[b])
        full = np.concatenate((cf["active_slots"], [gen_slot[b]]))
        positions = np.concatenate((cf["active_positions"], [lay.next_position]))
        q_pos = lay.next_position  # one generated token
        visible = full[q_pos - positions <= window]
        np.testing.assert_array_equal(full_ix[full_ip[b] : full_ip[b + 1]], full)
        np.testing.assert_array_equal(win_ix[win_ip[b] : win_ip[b + 1]], visible)
        assert len(visible) == window + 1
        for layer in range(model.n_layers):
            keys = visible if layer % 2 == 0 else full
            sel = torch.from_numpy(keys.astype(np.int64)).to(device)
            kk, vv = _f32(pool.k[layer][sel]), _f32(pool.v[layer][sel])
            want = oat.decode_attention(qq[b], kk, vv, 0.125, _f32(sinks[layer]))
            err = np.abs(_f32(outs[layer][b]) - want).max()
            assert err <= TOL, f"request {b} layer {layer}: max err {err}"
    del pool, outs
    torch.cuda.empty_cache()  # the 144 GiB pool
