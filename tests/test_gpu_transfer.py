"""GPU checks of the all-layer KV row copy (compacted handoff): pack ->
unpack round trip, direct pool-to-pool copy and padded slot strides, all
bit for bit against torch gathers of the same rows."""

import numpy as np
import pytest
import torch

from akv_amd import transfer

pytestmark = pytest.mark.gpu


def _pool(device, layers, slots, heads, dim, seed, pad=0):
    g = torch.Generator(device=device).manual_seed(seed)
    ks, vs = [], []
    for _ in range(layers):
        for store in (ks, vs):
            base = torch.randn((slots, heads * dim + pad), generator=g, device=device).to(torch.bfloat16)
            store.append(base[:, : heads * dim].view(slots, heads, dim) if pad else base.view(slots, heads, dim))
    ptr = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.uint64, device=device)
    return ks, vs, ptr(ks), ptr(vs)


def _bits(t):
    return t.view(torch.int16)


def test_pack_unpack_round_trip(device):
    layers, slots, heads, dim = 6, 30000, 8, 64
    ks, vs, kp, vp = _pool(device, layers, slots, heads, dim, seed=1)
    rng = np.random.default_rng(1)
    active = torch.from_numpy(rng.choice(np.arange(1, slots), size=5000, replace=False).astype(np.int32)).to(device)
    packed = transfer.PackedKV.empty(layers, 5000, heads, dim, torch.bfloat16, device)
    transfer.pack_active_kv(kp, vp, ks[0], active, packed)
    torch.cuda.synchronize()
    for l in range(layers):
        assert torch.equal(_bits(packed.k[l]), _bits(ks[l][active.long()]))
        assert torch.equal(_bits(packed.v[l]), _bits(vs[l][active.long()]))
    # D side: a second pool receives the rows at freshly allocated owners
    ks2, vs2, kp2, vp2 = _pool(device, layers, 12000, heads, dim, seed=2)
    before_k = [t.clone() for t in ks2]
    dest = torch.from_numpy(rng.choice(np.arange(1, 12000), size=5000, replace=False).astype(np.int32)).to(device)
    transfer.unpack_active_kv(packed, kp2, vp2, ks2[0], dest)
    torch.cuda.synchronize()
    untouched = torch.ones(12000, dtype=torch.bool, device=device)
    untouched[dest.long()] = False
    for l in range(layers):
        assert torch.equal(_bits(ks2[l][dest.long()]), _bits(ks[l][active.long()]))
        assert torch.equal(_bits(vs2[l][dest.long()]), _bits(vs[l][active.long()]))
        assert torch.equal(_bits(ks2[l][untouched]), _bits(before_k[l][untouched]))


def test_direct_pool_to_pool_with_padded_strides(device):
    layers, heads, dim = 3, 4, 128
    ks, vs, kp, vp = _pool(device, layers, 4000, heads, dim, seed=3, pad=64)
    ks2, vs2, kp2, vp2 = _pool(device, layers, 5000, heads, dim, seed=4)
    rng = np.random.default_rng(3)
    src = torch.from_numpy(rng.choice(4000, size=777, replace=False).astype(np.int32)).to(device)
    dst = torch.from_numpy(rng.choice(5000, size=777, replace=False).astype(np.int32)).to(device)
    transfer.copy_kv_rows(kp, vp, ks[0], kp2, vp2, ks2[0], 777, src_slots=src, dst_slots=dst)
    torch.cuda.synchronize()
    for l in range(layers):
        assert torch.equal(_bits(ks2[l][dst.long()]), _bits(ks[l][src.long()]))
        assert torch.equal(_bits(vs2[l][dst.long()]), _bits(vs[l][src.long()]))


def test_validation(device):
    ks, vs, kp, vp = _pool(device, 2, 100, 2, 64, seed=5)
    odd = torch.zeros((100, 2, 63), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="contiguous heads|16-byte"):
        transfer.copy_kv_rows(kp, vp, odd, kp, vp, ks[0], 4)
    with pytest.raises(ValueError, match="int32"):
        transfer.copy_kv_rows(kp, vp, ks[0], kp, vp, ks[0], 4, src_slots=torch.zeros(4, dtype=torch.int64,
                                                                                    device=device))


@pytest.mark.parametrize("layers,heads,dim", [(37, 8, 64), (5, 1, 8), (4, 3, 40), (3, 1, 264), (3, 16, 128),
                                               (2, 1, 1024), (2, 8, 1024)])
def test_row_sizes_and_layer_counts(device, layers, heads, dim):
    """Rows of 64, 1, 15, 33, 256, 128 and 1024 16-byte chunks: the
    layer-major kernel with several rows per wave (1 and 15 chunks), one row
    per wave with one to eight chunks per lane (33 to 512 chunks), and the
    flat kernel (longer rows) copy the same rows."""
    slots = 3000
    ks, vs, kp, vp = _pool(device, layers, slots, heads, dim, seed=layers + dim)
    ks2, vs2, kp2, vp2 = _pool(device, layers, slots, heads, dim, seed=layers + dim + 1)
    rng = np.random.default_rng(dim)
    n = 1234
    src = torch.from_numpy(rng.choice(slots, size=n, replace=False).astype(np.int32)).to(device)
    dst = torch.from_numpy(rng.choice(slots, size=n, replace=False).astype(np.int32)).to(device)
    before = [t.clone() for t in vs2]
    transfer.copy_kv_rows(kp, vp, ks[0], kp2, vp2, ks2[0], n, src_slots=src, dst_slots=dst)
    torch.cuda.synchronize()
    untouched = torch.ones(slots, dtype=torch.bool, device=device)
    untouched[dst.long()] = False
    for l in range(layers):
        assert torch.equal(_bits(ks2[l][dst.long()]), _bits(ks[l][src.long()])), f"layer {l} K"
        assert torch.equal(_bits(vs2[l][dst.long()]), _bits(vs[l][src.long()])), f"layer {l} V"
        assert torch.equal(_bits(vs2[l][untouched]), _bits(before[l][untouched])), f"layer {l} V untouched"


@pytest.mark.parametrize("seed", range(10))
def test_random_copies(device, seed):
    # seeded random geometry: layers, heads, head dims (rows of 1 to 512
    # 16-byte chunks), padded source strides, copy counts
    rng = np.random.default_rng(1200 + seed)
    layers = int(rng.integers(1, 41))
    heads = int(rng.choice([1, 2, 3, 4, 8]))
    dim = int(rng.choice([8, 16, 24, 40, 64, 128, 256]))
    pad = int(rng.choice([0, 0, 8, 64]))
    slots = int(rng.integers(200, 4000))
    n = int(rng.integers(1, slots // 2))
    print(f"transfer random {seed}: layers={layers} heads={heads} dim={dim} pad={pad} slots={slots} n={n}", flush=True)
    ks, vs, kp, vp = _pool(device, layers, slots, heads, dim, seed=1200 + seed, pad=pad)
    ks2, vs2, kp2, vp2 = _pool(device, layers, slots, heads, dim, seed=1300 + seed)
    src = torch.from_numpy(rng.choice(slots, size=n, replace=False).astype(np.int32)).to(device)
    dst = torch.from_numpy(rng.choice(slots, size=n, replace=False).astype(np.int32)).to(device)
    before_k = [t.clone() for t in ks2]
    transfer.copy_kv_rows(kp, vp, ks[0], kp2, vp2, ks2[0], n, src_slots=src, dst_slots=dst)
    torch.cuda.synchronize()
    untouched = torch.ones(slots, dtype=torch.bool, device=device)
    untouched[dst.long()] = False
    for l in range(layers):
        assert torch.equal(_bits(ks2[l][dst.long()]), _bits(ks[l][src.long()])), f"layer {l} K"
        assert torch.equal(_bits(vs2[l][dst.long()]), _bits(vs[l][src.long()])), f"layer {l} V"
        assert torch.equal(_bits(ks2[l][untouched]), _bits(before_k[l][untouched])), f"layer {l} K untouched"
