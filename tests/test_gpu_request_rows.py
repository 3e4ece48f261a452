"""GPU: per-request rows and overflow side rows (``akv_amd.request_rows``):
a side row appears only for a Context request that outgrows the pool row,
its device address replaces the pool row's in the pointer table, batched
writes reach pool rows and side rows alike (``akv_write_row_slots``), and a
release restores the pool row's address."""

from types import SimpleNamespace

import pytest
import torch

from akv_amd import request_rows as rr

pytestmark = pytest.mark.gpu


def _req(idx, prompt, budget, context=True):
    return SimpleNamespace(context_program=object() if context else None, origin_input_ids=[0] * prompt,
                           sampling_params=SimpleNamespace(max_new_tokens=budget),
                           kv=SimpleNamespace(req_pool_idx=idx))


def test_side_rows_pointers_and_writes(device):
    table = torch.full((4, 16), -7, dtype=torch.int32, device=device)
    pool = SimpleNamespace(req_to_token=table, device=device)
    rr.prepare_request_row(pool, _req(0, 5, 3))          # fits: no side row
    rr.prepare_request_row(pool, _req(1, 40, 8, False))  # ordinary request: never
    assert rr.row_pointers(pool) is None
    rr.prepare_request_row(pool, _req(2, 20, 10))        # 34 > 16: side row
    side = rr.request_row(pool, 2)
    assert side.numel() == 34 and bool((side == -1).all())
    ptrs = rr.row_pointers(pool)
    want = [table[i].data_ptr() for i in range(4)]
    want[2] = side.data_ptr()
    assert ptrs.cpu().tolist() == want
    with pytest.raises(RuntimeError, match="cannot grow"):
        rr.prepare_request_row(pool, _req(2, 30, 10))
    # batched writes: rows 0, 2 (side, past the pool width), 3
    rows = torch.tensor([0, 2, 2, 3], dtype=torch.int64, device=device)
    cols = torch.tensor([1, 3, 30, 15], dtype=torch.int64, device=device)
    vals = torch.tensor([11, 22, 33, 44], dtype=torch.int32, device=device)
    rr.write_request_slots(pool, (rows, cols), vals)
    rr.write_request_slots(pool, (2, slice(0, 2)), torch.tensor([5, 6], dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert int(table[0, 1]) == 11 and int(table[3, 15]) == 44
    assert side[:4].cpu().tolist() == [5, 6, -1, 22] and int(side[30]) == 33
    assert int(table[2, 3]) == -7  # the pool row of a side-row request is untouched
    rr.release_request_row(pool, 2)
    assert rr.row_pointers(pool) is None
    assert pool._context_row_pointers[2].item() == table[2].data_ptr()
    rr.write_request_slots(pool, (rows[:1], cols[:1]), vals[1:2])  # no side rows left: plain indexing
    assert int(table[0, 1]) == 22
