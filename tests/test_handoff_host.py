"""Host logic of the P -> D handoff mirror (``akv_amd.handoff``) against
independent loop models: the transfer signature (blake2b of the event
identity, recomputed here with hashlib), the SWA start, chunking of a
completed raw range, active lengths, the missing-page filter and D's reuse
decision."""

import hashlib
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import ownership_scenarios as scenarios
from akv_amd import handoff, plan

INF = 2**31 - 1


def _program(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(20, 90))
    while True:
        events, visible = scenarios._program(rng, n)
        t = {k: torch.from_numpy(np.asarray(v)).to(torch.int32) for k, v in events.items()}
        try:
            lay = plan.compile_context_layout(**t)
            break
        except ValueError:
            continue
    return SimpleNamespace(layout=lay, visible_until=torch.from_numpy(np.minimum(visible, INF).astype(np.int32))), rng


def test_plan_identity_and_swa_start():
    for seed in range(30):
        prog, rng = _program(seed)
        p = handoff.ContextTransferPlan.build(prog, torch.device("cpu"))
        h = hashlib.blake2b(digest_size=8)
        for a in (prog.layout.records, prog.layout.keep_mask, prog.visible_until):
            h.update(a.numpy().tobytes())
        assert p.signature == tuple(int(x) for x in np.frombuffer(h.digest(), dtype="<i4"))
        keep = prog.layout.keep_mask.numpy()
        assert p.active_count == int(keep.sum())
        assert p.header() == (2, p.active_count, prog.layout.next_position, *p.signature)
        pos = prog.layout.positions.numpy()[keep]
        for window in (0, 1, 5, 40, 1000):
            lower = prog.layout.next_position - window
            assert p.swa_start(window) == sum(1 for x in pos if x < lower)
        # another keep mask is another identity
        flipped = prog.layout.keep_mask.clone()
        flipped[0] = ~flipped[0]
        other = SimpleNamespace(layout=SimpleNamespace(**{**vars(prog.layout), "keep_mask": flipped}),
                                visible_until=prog.visible_until)
        h2 = hashlib.blake2b(digest_size=8)
        for a in (other.layout.records, other.layout.keep_mask, other.visible_until):
            h2.update(a.numpy().tobytes())
        assert h2.digest() != h.digest()


def _chunk_model(raw, raw_start, raw_end, last_chunk, terminal=None, owned=None):
    """Loop model: send the active versions of [raw_start, raw_end) in order,
    stop (non-final) at the first without a stable terminal owner, withhold
    the last active version until the final send; the cursor stops at the
    first version not sent."""
    begin = sum(1 for r in raw if r < raw_start)
    end = begin
    while end < len(raw) and raw[end] < raw_end:
        if terminal is not None:
            row = terminal[raw[end]]
            if last_chunk and row < 0:
                raise ValueError("missing")
            if not last_chunk and (row < 0 or (owned is not None and owned[row])):
                break
        end += 1
    if not last_chunk:
        end = min(end, max(0, len(raw) - 1))
    cursor = raw_end if end >= len(raw) else min(raw_end, raw[end])
    return begin, end, cursor


def test_full_chunk_against_loop_model():
    for seed in range(40):
        prog, rng = _program(100 + seed)
        p = handoff.ContextTransferPlan.build(prog, torch.device("cpu"))
        raw = p.decode.raw_indices.tolist()
        n = len(prog.layout.positions)
        rows = np.where(rng.random(n) < 0.8, np.arange(n), -1).astype(np.int64)
        owned = rng.random(n) < 0.2
        for _ in range(10):
            a = int(rng.integers(0, n))
            b = int(rng.integers(a, n + 1))
            for last in (False, True):
                assert p.full_chunk(a, b, last_chunk=last) == _chunk_model(raw, a, b, last)
                try:
                    want = _chunk_model(raw, a, b, last, rows, owned)
                except ValueError:
                    with pytest.raises(ValueError, match="missing terminal KV"):
                        p.full_chunk(a, b, last_chunk=last, terminal_rows=torch.from_numpy(rows),
                                     owned=torch.from_numpy(owned))
                    continue
                assert p.full_chunk(a, b, last_chunk=last, terminal_rows=torch.from_numpy(rows),
                                    owned=torch.from_numpy(owned)) == want


def test_active_lengths_and_missing_filter():
    for seed in range(20):
        prog, rng = _program(200 + seed)
        p = handoff.ContextTransferPlan.build(prog, torch.device("cpu"))
        req = SimpleNamespace(context_decode_layout=p.decode)
        n = len(prog.layout.positions)
        pos = p.decode.positions
        for generated in (0, 1, 7):
            for window in (1, 4, 30, 500):
                full, win = handoff.request_active_lengths(req, n + generated, window)
                assert full == len(pos) + generated
                lower = p.decode.next_position + generated - window
                assert win == sum(1 for x in pos if x >= lower) + min(generated, window)
    src, dst = np.arange(10), np.arange(100, 110)
    reuse = np.zeros(10, dtype=bool)
    reuse[[1, 4, 5]] = True
    s, d = handoff.select_missing_transfer(src, dst, reuse)
    assert s.tolist() == [0, 2, 3, 6, 7, 8, 9] and d.tolist() == [100, 102, 103, 106, 107, 108, 109]
    with pytest.raises(ValueError, match="must be boolean"):
        handoff.select_missing_transfer(src, dst, reuse.astype(np.int8))
    with pytest.raises(ValueError, match="disagree"):
        handoff.select_missing_transfer(src, dst[:5], reuse)


def test_decode_reuse_against_loop_model():
    for seed in range(40):
        prog, rng = _program(300 + seed)
        p = handoff.ContextTransferPlan.build(prog, torch.device("cpu"))
        n = len(prog.layout.positions)
        matched = int(rng.integers(0, n + 1))
        resident = torch.from_numpy(rng.random(matched) < 0.85) if rng.random() < 0.5 else None
        source = (torch.from_numpy(np.asarray(prog.layout.birth_positions.numpy()[:matched], np.int32))
                  if rng.random() < 0.5 else None)
        exact = int(rng.integers(0, matched + 1))
        window = int(rng.integers(1, 40)) if rng.random() < 0.5 else None
        req = SimpleNamespace(prefix_indices=torch.arange(1000, 1000 + matched), context_resident=resident,
                              context_source_positions=source, context_exact_prefix_len=exact)
        got = handoff.ContextDecodeReuse.build(req, p, window=window)
        raw, pos = p.decode.raw_indices, p.decode.positions
        swa0 = p.swa_start(window) if window is not None else len(raw)
        src_pos = source.numpy() if source is not None else np.arange(matched)
        want_reuse, want_borrow, want_copy, want_pairs = [], [], [], []
        for i, r in enumerate(raw.tolist()):
            ok = r < matched and (resident is None or bool(resident[r])) and i < swa0
            want_reuse.append(ok)
            moves = ok and (int(src_pos[r]) != int(pos[i]) or r >= exact)
            want_borrow.append(ok and not moves)
            if moves:
                want_copy.append(i)
                want_pairs.append((int(src_pos[r]), int(pos[i])))
        assert got.reusable.tolist() == want_reuse
        assert got.borrowed.tolist() == want_borrow
        assert got.copy_indices.tolist() == want_copy
        assert [tuple(x) for x in got.position_pairs.tolist()] == want_pairs
        assert got.allocation_count == len(raw) - sum(want_borrow)
