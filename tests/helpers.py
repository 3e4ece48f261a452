"""Shared helpers of the GPU parity tests (torch <-> oracle storage)."""

import numpy as np
import torch

from akv_amd import synth

ORACLE_DTYPE = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def to_storage(t):
    """torch tensor -> numpy storage array the oracle reads (bits for 16-bit types)."""
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.contiguous().numpy()


def storage_equal(a, b):
    return np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


def single_request(name, device):
    """Layout, slots and device inputs of a one-request synthetic workload."""
    w = synth.workload(name)
    layout = synth.compile_layouts(w)[0]
    slots = synth.assign_slots(w, [layout])
    moved = layout.keep_mask & (layout.birth_positions != layout.positions)
    birth = slots.birth_rows[0]
    fresh = slots.fresh[0]
    src = birth[moved.numpy()].astype(np.int32)
    pairs = np.stack((layout.birth_positions.numpy()[moved.numpy()], layout.positions.numpy()[moved.numpy()]), 1)
    return dict(
        workload=w,
        layout=layout,
        birth=birth,
        fresh=fresh,
        src=torch.from_numpy(src).to(device),
        dst=torch.from_numpy(fresh.astype(np.int32)).to(device),
        pairs=torch.from_numpy(pairs.astype(np.int32)).to(device),
    )
