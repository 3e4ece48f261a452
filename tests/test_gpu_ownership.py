"""GPU: the ownership planner with its device gather (``akv_gather_slots``)
against the golden traces of the reference module, bit for bit; one
batched advance of many requests equals their one-by-one advances; the
plan's ``bind`` agrees with the advance on every bound occurrence."""

import numpy as np
import pytest
import torch

import ownership_scenarios as scenarios
from akv_amd import ownership
from golden import ownership_vectors as vectors

pytestmark = pytest.mark.gpu


def _same(a, b):
    if a is None or b is None:
        return a is None and b is None
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.astype(np.int64), b.astype(np.int64))


@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_lifecycles_match_reference_traces(device, slot_dtype):
    golden = vectors.unpack(np.load(vectors.OUT))
    impl = scenarios.NativeImpl(device, slot_dtype)
    print(f"ownership lifecycles, slots {slot_dtype}", flush=True)
    for seed in vectors.SEEDS:
        want = golden[seed]
        got = scenarios.run(scenarios.make(seed), impl)
        torch.cuda.synchronize()
        assert [k for k, _ in got] == [k for k, _ in want], seed
        for (name, a), (_, b) in zip(got, want):
            assert _same(a, b), (seed, name)


def _first_forward(seed, impl, slot_base):
    """State, window, plan and slots of a scenario's first forward."""
    sc = scenarios.make(seed)
    mt = sc["match"]
    m = mt["length"]
    st = impl.from_match(mt["slots"][:m], mt["positions"][:m], mt["exact"], mt["resident"][:m],
                         None if mt["swa"] is None else mt["swa"][:m])
    qs, qe = sc["forwards"][0], sc["forwards"][1]
    win = impl.window(sc["layout"], sc["visible"], qs, qe)
    keep = impl.keep(st, sc["layout"], qe)
    try:
        p = impl.plan(st, win, keep)
    except ValueError:
        return None
    q = impl._slots(slot_base + np.arange(qe - qs))
    extra = impl._slots(slot_base + 10_000 + np.arange(p["extra_page_count"]))
    vis = torch.from_numpy(sc["visible"])
    return st, win["_obj"], p["_obj"], q, extra, vis


def test_batched_advance_equals_one_by_one(device):
    impl = scenarios.NativeImpl(device)
    steps = []
    for seed in range(60):
        s = _first_forward(seed, impl, 100_000 * (seed + 1))
        if s is not None:
            steps.append(s)
    assert len(steps) > 40
    print(f"batched advance of {len(steps)} requests", flush=True)
    results, batch = ownership.advance_batch(steps)
    torch.cuda.synchronize()
    occ, src, dst, pairs = [], [], [], []
    for step, got in zip(steps, results):
        want = step[0].advance(*step[1:])
        for name in ("occurrence_slots", "copy_source_slots", "copy_destination_slots", "copy_position_pairs",
                     "retired_slots", "unused_swa_slots", "retired_swa_resident"):
            a, b = getattr(got, name), getattr(want, name)
            assert (a is None) == (b is None) and (a is None or torch.equal(a.cpu(), b.cpu())), name
        assert torch.equal(got.state.slots.cpu(), want.state.slots.cpu())
        assert torch.equal(got.state.canonical_rows, want.state.canonical_rows)
        occ.append(want.occurrence_slots)
        src.append(want.copy_source_slots)
        dst.append(want.copy_destination_slots)
        pairs.append(want.copy_position_pairs)
    assert torch.equal(batch.occurrence_slots, torch.cat(occ))
    assert torch.equal(batch.copy_source_slots, torch.cat(src))
    assert torch.equal(batch.copy_destination_slots, torch.cat(dst))
    assert torch.equal(batch.copy_position_pairs, torch.cat(pairs))


def test_plan_bind_agrees_with_advance(device):
    impl = scenarios.NativeImpl(device)
    checked = 0
    for seed in range(40):
        s = _first_forward(seed, impl, 1000)
        if s is None:
            continue
        st, win, p, q, extra, vis = s
        n = len(win.birth_occurrences)
        start = len(st.canonical_rows)
        slots = st.slots.cpu().numpy()
        canonical = np.full(n, 0, dtype=np.int64)
        rows = st.canonical_rows.numpy()
        canonical[:start][rows >= 0] = slots[rows[rows >= 0]]
        canonical[start : start + len(q)] = q.cpu().numpy()
        terminal = np.zeros(n, dtype=np.int64)
        trows = st.terminal_rows.numpy()
        terminal[:start][trows >= 0] = slots[trows[trows >= 0]]
        bound, bsrc, bdst, bpairs = p.bind(impl._slots(canonical), impl._slots(terminal), extra)
        adv = st.advance(win, p, q, extra, vis)
        torch.cuda.synchronize()
        b = bound.cpu().numpy()
        ok = p.source_rows.numpy() >= 0
        ok[p.allocated_occurrences.numpy()] = True
        assert np.array_equal(b[ok], adv.occurrence_slots.cpu().numpy()[ok]), seed
        assert np.all(b[~ok] == -1)
        assert torch.equal(bsrc.cpu(), adv.copy_source_slots.cpu())
        assert torch.equal(bdst.cpu(), adv.copy_destination_slots.cpu())
        assert torch.equal(bpairs.cpu(), adv.copy_position_pairs.cpu())
        checked += 1
    assert checked > 25


def test_long_lifecycles_match_the_oracle(device):
    """Prompts of 300-1500 tokens, up to 12 turns and 8 forwards, through the
    HIP gather: the trace equals the oracle's."""
    native = scenarios.NativeImpl(device)
    oracle = scenarios.OracleImpl()
    print("long ownership lifecycles", flush=True)
    for seed in range(30):
        sc = scenarios.make(5000 + seed, n_range=(300, 1500), max_cuts=8)
        want = scenarios.run(sc, oracle)
        got = scenarios.run(sc, native)
        torch.cuda.synchronize()
        assert [k for k, _ in got] == [k for k, _ in want], seed
        for (name, a), (_, b) in zip(got, want):
            assert _same(a, b), (seed, name)
