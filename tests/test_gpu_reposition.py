"""GPU parity of the fused Reposition kernel against the CPU oracle.

Bit-exact for K, V and every untouched slot, across dtypes, pair styles,
partial rotary widths, strides, pointer alignment, lists long enough to be
swept in token chunks, and the full 32k GPT-OSS shape (every destination
row of every layer against the torch-CPU restatement).
"""

import re

import numpy as np
import pytest
import torch

from akv_amd import ops, synth
from akv_amd.rope import make_table
from oracle import reposition as rp

from helpers import ORACLE_DTYPE, single_request, storage_equal, to_storage
from reposition_kat import kat_expected, kat_pool

pytestmark = pytest.mark.gpu


def _run_case(device, *, layers=2, heads=2, head_dim=64, rotary_dim=None, kv_dtype=torch.bfloat16,
              table_dtype=torch.float32, neox=True, slots=512, moved=200, seed=0, skip_unmapped=False,
              same_every=0, misalign=False, slot_stride_extra=0, table_kind="yarn", nonfinite=False):
    rotary_dim = rotary_dim or head_dim
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    width = head_dim * heads + slot_stride_extra
    k_store, v_store, k_views, v_views = [], [], [], []
    for _ in range(layers):
        # a wider backing buffer gives non-contiguous slot strides when
        # slot_stride_extra > 0, and a shifted base when misalign is set
        kb = torch.randn((slots * width + 16,), generator=g).to(kv_dtype)
        vb = torch.randn((slots * width + 16,), generator=g).to(kv_dtype)
        if nonfinite:
            _plant_nonfinite(kb, rng)
            _plant_nonfinite(vb, rng)
        kb, vb = kb.to(device), vb.to(device)
        off = 1 if misalign else 0
        k_views.append(kb[off : off + slots * width].view(slots, width)[:, : heads * head_dim].view(slots, heads, head_dim)
                       if slot_stride_extra == 0 else
                       torch.as_strided(kb, (slots, heads, head_dim), (width, head_dim, 1), off))
        v_views.append(vb[off : off + slots * width].view(slots, width)[:, : heads * head_dim].view(slots, heads, head_dim)
                       if slot_stride_extra == 0 else
                       torch.as_strided(vb, (slots, heads, head_dim), (width, head_dim, 1), off))
        k_store.append(kb)
        v_store.append(vb)
    perm = rng.permutation(np.arange(1, slots))
    src = perm[:moved].astype(np.int32)
    dst = perm[moved : 2 * moved].astype(np.int32)
    if skip_unmapped:
        src[::7] = 0
        dst[3::11] = -1
    positions = 300
    old = rng.integers(0, positions, size=moved)
    new = rng.integers(0, positions, size=moved)
    if same_every:
        new[::same_every] = old[::same_every]
    pairs = np.stack((old, new), 1).astype(np.int32)
    table = make_table(table_kind, rotary_dim, positions, base=150000.0, factor=32.0, original_max=4096) \
        if table_kind == "yarn" else make_table("plain", rotary_dim, positions, base=10000.0)
    table = table.to(table_dtype)

    k_np = [to_storage(t) for t in k_views]
    v_np = [to_storage(t) for t in v_views]
    rp.reposition_kv_layers(k_np, v_np, src, dst, pairs, to_storage(table), dtype=ORACLE_DTYPE[kv_dtype],
                            cos_sin_dtype=ORACLE_DTYPE[table_dtype], is_neox_style=neox,
                            skip_unmapped=skip_unmapped, rotary_dim=rotary_dim)
    k_ptrs = torch.tensor([t.data_ptr() for t in k_views], dtype=torch.uint64).to(device)
    v_ptrs = torch.tensor([t.data_ptr() for t in v_views], dtype=torch.uint64).to(device)
    ops.reposition_kv_layers(
        k_ptrs, v_ptrs, k_views[0], v_views[0],
        torch.from_numpy(src).to(device), torch.from_numpy(dst).to(device),
        torch.from_numpy(pairs).to(device), table.to(device),
        is_neox_style=neox, skip_unmapped=skip_unmapped, rotary_dim=rotary_dim,
    )
    torch.cuda.synchronize()
    for layer in range(layers):
        got_k, got_v = to_storage(k_views[layer]), to_storage(v_views[layer])
        if nonfinite:
            _assert_nan_aware(got_k, k_np[layer], ORACLE_DTYPE[kv_dtype], f"K layer {layer}")
            # rows whose pair keeps its position are stored as their source
            # bits, NaN payloads included (context_reposition.py:98-112)
            same = (pairs[:, 0] == pairs[:, 1]) & (src > 0) & (dst > 0)
            assert storage_equal(got_k[dst[same]], k_np[layer][dst[same]]), f"K layer {layer}: same-position rows"
            assert storage_equal(got_v, v_np[layer]), f"V layer {layer}"
            continue
        if not storage_equal(got_k, k_np[layer]):
            diff = np.argwhere(got_k != k_np[layer])
            raise AssertionError(f"K layer {layer}: {len(diff)} elements differ, first {diff[:5].tolist()}")
        assert storage_equal(got_v, v_np[layer]), f"V layer {layer}"


def _plant_nonfinite(buf, rng):
    """Sets ~3% of a KV buffer to +-inf and NaNs of several payloads (quiet,
    signalling, negative) in place."""
    n = buf.numel()
    idx = torch.from_numpy(rng.choice(n, n // 32, replace=False))
    if buf.dtype == torch.float32:
        pats = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFFC12345, 0x7FBFFFFF], dtype=np.uint32)
        bits = torch.from_numpy(pats[rng.integers(0, len(pats), len(idx))].view(np.int32))
        buf.view(torch.int32)[idx] = bits
    else:
        pats = (np.array([0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0xFFC5, 0x7FBF], dtype=np.uint16)
                if buf.dtype == torch.bfloat16 else
                np.array([0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE05, 0x7DFF], dtype=np.uint16))
        bits = torch.from_numpy(pats[rng.integers(0, len(pats), len(idx))].view(np.int16))
        buf.view(torch.int16)[idx] = bits


def _assert_nan_aware(got, want, dtype, what):
    """Bit-exact wherever the oracle's value is not a NaN; a NaN exactly where
    the oracle has one (the payload of a NaN that the rotation produces is the
    hardware's: the one part left open)."""
    from oracle.bf16 import to_f32

    g, w = to_f32(got, dtype), to_f32(want, dtype)
    gn, wn = np.isnan(g), np.isnan(w)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ ({int((gn != wn).sum())} elements)"
    assert storage_equal(np.asarray(got)[~wn], np.asarray(want)[~wn]), f"{what}: finite or infinite values differ"


@pytest.mark.filterwarnings("ignore:invalid value:RuntimeWarning", "ignore:overflow:RuntimeWarning")
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("neox", [True, False])
def test_nonfinite_inputs(device, kv_dtype, neox):
    """K and V rows holding +-inf and NaNs (quiet, signalling, negative
    payloads), with a third of the pairs at their own position: every value
    the oracle's IEEE arithmetic makes finite or infinite is bit-exact, NaNs
    land where the oracle's do, V and same-position rows keep their bits."""
    _run_case(device, kv_dtype=kv_dtype, neox=neox, seed=17, nonfinite=True, same_every=3)
    _run_case(device, kv_dtype=kv_dtype, neox=neox, rotary_dim=32, seed=18, nonfinite=True, same_every=3)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dtypes_and_styles(device, neox, kv_dtype):
    _run_case(device, kv_dtype=kv_dtype, neox=neox, seed=1)


@pytest.mark.parametrize("table_dtype", [torch.bfloat16, torch.float16])
def test_half_precision_tables(device, table_dtype):
    _run_case(device, table_dtype=table_dtype, seed=2)


@pytest.mark.parametrize("rotary_dim", [32, 16, 48])
def test_partial_rotary(device, rotary_dim):
    _run_case(device, rotary_dim=rotary_dim, seed=3)
    _run_case(device, rotary_dim=rotary_dim, neox=False, seed=4)


# (8, 64, 36) is the GPT-OSS geometry (32 lanes per row, 8 tokens per
# workgroup); (8, 128, 32) the Llama-3 one (64 lanes per row, 4 tokens);
# (4, 64, 36) one TP=2 rank's GPT-OSS share (16 lanes per row, 16 tokens);
# (1, 16, 2) and (3, 32, 2) rows narrower than a wave
@pytest.mark.parametrize("heads,head_dim,layers", [(8, 64, 36), (8, 128, 3), (8, 128, 32), (4, 64, 36), (4, 64, 5),
                                                   (1, 16, 2), (3, 32, 2)])
def test_shapes(device, heads, head_dim, layers):
    _run_case(device, heads=heads, head_dim=head_dim, layers=layers, moved=64, seed=5)


@pytest.mark.parametrize("neox", [True, False])
def test_exact_known_answers(device, neox):
    """The kernel against the exact-arithmetic known answers of the fp32
    operation order (each case tells the reference order apart from a
    delta-angle rotation, per-term division and fused multiply-adds)."""
    k, v, src, dst, pairs, table = kat_pool(neox)
    kt = torch.from_numpy(k[0].view(np.int16)).view(torch.bfloat16).to(device)
    vt = torch.from_numpy(v[0].view(np.int16)).view(torch.bfloat16).to(device)
    ptr = lambda t: torch.tensor([t.data_ptr()], dtype=torch.uint64).to(device)  # noqa: E731
    as_i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device)  # noqa: E731
    ops.reposition_kv_layers(ptr(kt), ptr(vt), kt, vt, as_i32(src), as_i32(dst), as_i32(pairs),
                             torch.from_numpy(table).to(device), is_neox_style=neox)
    torch.cuda.synchronize()
    got = to_storage(kt)
    np.testing.assert_array_equal(got[dst], kat_expected("two_step", neox))
    np.testing.assert_array_equal(to_storage(vt)[dst], v[0][src])
    untouched = np.setdiff1d(np.arange(len(got)), dst)
    np.testing.assert_array_equal(got[untouched], k[0][untouched])


@pytest.mark.parametrize("heads,head_dim,layers,moved", [(8, 64, 4, 40003), (8, 128, 3, 17001)])
def test_chunked_sweep(device, heads, head_dim, layers, moved):
    """Lists whose cos/sin rows pass 16 MiB (32768 tokens of a 64-dim fp32
    table, 16384 of a 128-dim one) are swept in 1024-token chunks: odd
    counts leave a partial last block and padding blocks in the last, shorter
    chunk.  Unmapped entries and same-position pairs mixed in."""
    print(f"chunked sweep {heads}x{head_dim}, {layers} layers, {moved} tokens", flush=True)
    _run_case(device, layers=layers, heads=heads, head_dim=head_dim, slots=2 * moved + 8, moved=moved, seed=11,
              skip_unmapped=True, same_every=5)


def test_skip_unmapped_and_same_position(device):
    _run_case(device, skip_unmapped=True, same_every=3, seed=6)


def test_misaligned_and_strided_layers(device):
    _run_case(device, misalign=True, seed=7)  # element-wise path inside the vector kernel
    _run_case(device, slot_stride_extra=8, seed=8)
    _run_case(device, slot_stride_extra=3, seed=9)  # generic kernel (odd stride)


def test_odd_rotary_goes_generic(device):
    _run_case(device, head_dim=40, rotary_dim=10, seed=10, table_kind="plain")


@pytest.mark.parametrize("seed", range(16))
def test_random_cases(device, seed):
    # seeded random geometry and options: layers, heads, head_dim, partial
    # rotary widths, KV and table dtypes, pair style, table kind, unmapped
    # and same-position pairs, misaligned bases and padded slot strides
    rng = np.random.default_rng(900 + seed)
    head_dim = int(rng.choice([16, 32, 40, 64, 128]))
    rotary_dim = int(rng.choice([head_dim, head_dim, 2 * int(rng.integers(1, head_dim // 2 + 1))]))
    moved = int(rng.integers(1, 300))
    case = dict(layers=int(rng.integers(1, 41)), heads=int(rng.choice([1, 2, 3, 4, 8])), head_dim=head_dim,
                rotary_dim=rotary_dim, kv_dtype=[torch.bfloat16, torch.float16, torch.float32][rng.integers(0, 3)],
                table_dtype=[torch.float32, torch.bfloat16, torch.float16][rng.integers(0, 3)],
                neox=bool(rng.integers(0, 2)), slots=2 * moved + int(rng.integers(2, 200)), moved=moved,
                seed=900 + seed, skip_unmapped=bool(rng.random() < 0.3), same_every=int(rng.choice([0, 0, 2, 5])),
                misalign=bool(rng.random() < 0.2), slot_stride_extra=int(rng.choice([0, 0, 0, 8, 3])),
                table_kind=str(rng.choice(["yarn", "plain"])))
    if case["misalign"]:
        case["slot_stride_extra"] = 0
    print(f"reposition random {seed}: " + ", ".join(f"{k}={v}" for k, v in case.items()), flush=True)
    _run_case(device, **case)


def test_tiny_workload_bit_exact(device):
    case = single_request("tiny", device)
    w = case["workload"]
    pool = synth.make_pool(w.model, w.pool_slots, device, seed=0, generate_on_device=False)
    table = synth.rope_table(w, device)
    k_np = [to_storage(t) for t in pool.k]
    v_np = [to_storage(t) for t in pool.v]
    rp.reposition_kv_layers(k_np, v_np, case["src"].cpu().numpy(), case["dst"].cpu().numpy(),
                            case["pairs"].cpu().numpy(), to_storage(table), dtype="bf16")
    ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], case["src"], case["dst"],
                             case["pairs"], table)
    torch.cuda.synchronize()
    for l in range(w.model.n_layers):
        assert storage_equal(to_storage(pool.k[l]), k_np[l])
        assert storage_equal(to_storage(pool.v[l]), v_np[l])


# the headline request (12064 moved tokens) and the same shape at the median
# moved count over drop-span seeds (18192)
@pytest.mark.parametrize("name", ["gpt-oss-32k", "gpt-oss-32k-median"])
def test_gpt_oss_32k_full_size(device, name):
    """Every destination row of every layer, K and V, bit-exact against the
    torch-CPU restatement (itself pinned by the known answers), and every
    other slot of the pool unchanged."""
    from oracle import cpu_torch

    print(f"reposition full size {name}", flush=True)
    case = single_request(name, device)
    w = case["workload"]
    pool = synth.make_pool(w.model, w.pool_slots, device, seed=0)
    table = synth.rope_table(w, device)
    src, dst, pairs = case["src"], case["dst"], case["pairs"]
    m = len(src)
    # the source rows of every layer, before the Reposition, packed as slots
    # [0, m) of host buffers whose slots [m, 2m) receive the oracle's result
    host_k = [torch.cat((t[src.long()].cpu(), torch.zeros_like(t[src.long()].cpu()))) for t in pool.k]
    host_v = [torch.cat((t[src.long()].cpu(), torch.zeros_like(t[src.long()].cpu()))) for t in pool.v]
    # checksum of everything but the destination rows
    mask = torch.ones(w.pool_slots, dtype=torch.bool, device=device)
    mask[dst.long()] = False
    keep_sum = [t[mask].view(torch.int16).to(torch.int64).sum().item() for t in pool.k + pool.v]
    ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], src, dst, pairs, table)
    torch.cuda.synchronize()
    # nothing outside the destinations changed
    after_sum = [t[mask].view(torch.int16).to(torch.int64).sum().item() for t in pool.k + pool.v]
    assert after_sum == keep_sum
    cpu_torch.reposition_kv_layers(host_k, host_v, np.arange(m), np.arange(m, 2 * m), pairs.cpu().numpy(),
                                   table.cpu(), is_neox_style=w.model.is_neox_style)
    for l in range(w.model.n_layers):
        got_k = pool.k[l][dst.long()].cpu()
        got_v = pool.v[l][dst.long()].cpu()
        assert torch.equal(got_k.view(torch.int16), host_k[l][m:].view(torch.int16)), f"K layer {l}"
        assert torch.equal(got_v.view(torch.int16), host_v[l][m:].view(torch.int16)), f"V layer {l}"


def test_validation_messages(device):
    k = torch.zeros((8, 2, 64), dtype=torch.bfloat16, device=device)
    ptr = torch.tensor([k.data_ptr()], dtype=torch.uint64, device=device)
    s = torch.zeros(1, dtype=torch.int32, device=device)
    p = torch.zeros((1, 2), dtype=torch.int32, device=device)
    t = torch.zeros((4, 64), dtype=torch.float32, device=device)
    ok = dict(k_data_ptrs=ptr, v_data_ptrs=ptr, k_layout=k, v_layout=k, source_slots=s,
              destination_slots=s, position_pairs=p, cos_sin_cache=t)
    cases = [
        (dict(k_layout=k.to(torch.int8)), "Context Reposition requires unquantized floating-point KV"),
        (dict(v_layout=k[:, :1]), "Reposition requires matching native NHD K/V layouts"),
        (dict(k_layout=k.transpose(1, 2).contiguous().transpose(1, 2), v_layout=k.transpose(1, 2).contiguous().transpose(1, 2)),
         "Reposition requires contiguous head dimensions"),
        (dict(k_data_ptrs=ptr.to(torch.int32)), "Reposition requires contiguous 64-bit layer pointer tables"),
        (dict(source_slots=s.long()), "Reposition requires int32 slot vectors and [N, 2] positions"),
        (dict(position_pairs=p[:, :1]), "Reposition requires int32 slot vectors and [N, 2] positions"),
        (dict(cos_sin_cache=t[:, :32]), "Reposition requires a native cos/sin cache matching rotary_dim"),
        (dict(cos_sin_cache=t.cpu()), "Reposition tensors must be on one CUDA device"),
    ]
    for change, message in cases:
        args = dict(ok)
        args.update(change)
        with pytest.raises(ValueError, match=re.escape(message)):
            ops.reposition_kv_layers(**args)
    with pytest.raises(ValueError, match="Context Reposition requires page_size=1"):
        ops.reposition_kv_layers(**ok, page_size=16)
    # empty work returns without a launch
    ops.reposition_kv_layers(**dict(ok, source_slots=s[:0], destination_slots=s[:0], position_pairs=p[:0]))
