"""Host ownership planner (C++: ``akv_plan_ownership`` /
``akv_advance_ownership``) and the Python mirror of ``OccurrenceState``
against the golden traces of the reference module, on the CPU.

The device gather (``akv_gather_slots``) is replaced here by a numpy
statement of its contract -- element i = slot of rows[i] in its request's
concatenated pieces, -1 for row -1 -- so every host decision, segment and
state transition is checked without a GPU; ``tests/test_gpu_ownership.py``
runs the same traces through the HIP kernel."""

import numpy as np
import pytest
import torch

import ownership_scenarios as scenarios
from akv_amd import ownership
from golden import ownership_vectors as vectors


def _gather_on_cpu(self, extra_i32=()):
    pieces = [np.concatenate([p.numpy().astype(np.int64) for p in req if p is not None] or [np.zeros(0, np.int64)])
              for req in self.requests]

    def resolve(b, rows):
        out = np.full(len(rows), -1, dtype=np.int64)
        ok = rows >= 0
        assert np.all(rows[ok] < len(pieces[b])), "owner row beyond the request's slots"
        out[ok] = pieces[b][rows[ok]]
        return out

    wide = [torch.from_numpy(resolve(b, r)).to(self.dtype) for b, r in self.wide]
    narrow = [torch.from_numpy(resolve(b, r).astype(np.int32)) for b, r in self.narrow]
    extra = [torch.from_numpy(np.ascontiguousarray(e, dtype=np.int32).reshape(-1)) for e in extra_i32]
    return wide, narrow, extra


@pytest.fixture
def cpu_gather(monkeypatch):
    monkeypatch.setattr(ownership._Gather, "run", _gather_on_cpu)


def _same(a, b):
    if a is None or b is None:
        return a is None and b is None
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.astype(np.int64), b.astype(np.int64))


@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_lifecycles_match_reference_traces(cpu_gather, slot_dtype):
    golden = vectors.unpack(np.load(vectors.OUT))
    impl = scenarios.NativeImpl(torch.device("cpu"), slot_dtype)
    for seed in vectors.SEEDS:
        want = golden[seed]
        got = scenarios.run(scenarios.make(seed), impl)
        assert [k for k, _ in got] == [k for k, _ in want], seed
        for (name, a), (_, b) in zip(got, want):
            assert _same(a, b), (seed, name)


def test_direct_plans_match_reference(cpu_gather):
    golden = vectors.unpack(np.load(vectors.OUT))
    impl = scenarios.NativeImpl(torch.device("cpu"))
    for seed in vectors.SEEDS:
        got = scenarios.run_plan_case(scenarios.plan_case(seed), impl)
        want = golden[vectors.PLAN_CASES + seed]
        assert [k for k, _ in got] == [k for k, _ in want], seed
        for (name, a), (_, b) in zip(got, want):
            assert _same(a, b), (seed, name)


def test_reference_messages(cpu_gather):
    impl = scenarios.NativeImpl(torch.device("cpu"))
    sc = scenarios.make(3)
    lay = scenarios.torch_layout(sc["layout"])
    n = sc["n"]
    win = impl.window(sc["layout"], sc["visible"], 2, n)["_obj"]
    z = torch.zeros(2, dtype=torch.bool)
    pos = lay.positions[:2].clone()
    keep = torch.ones(n, dtype=torch.bool)
    with pytest.raises(ValueError, match="Invalid occurrence ownership/query boundaries"):
        ownership.plan_occurrence_materialization(win, pos, z, z, z, keep, query_start=2, query_end=n,
                                                  exact_prefix_len=3)
    with pytest.raises(ValueError, match="aligned CPU metadata"):
        ownership.plan_occurrence_materialization(win, pos.long(), z, z, z, keep, query_start=2, query_end=n,
                                                  exact_prefix_len=0)
    with pytest.raises(ValueError, match="does not cover the planned queries"):
        ownership.plan_occurrence_materialization(win, pos, z, z, z, keep[:-1], query_start=2, query_end=n - 1,
                                                  exact_prefix_len=0)
    st = impl.from_match(np.arange(2), sc["layout"].positions[:2], 2, np.ones(2, dtype=bool), None)
    p = st.plan(win, torch.from_numpy(impl.keep(st, sc["layout"], n)))
    with pytest.raises(ValueError, match="Context admission does not cover the selected window"):
        st.advance(win, p, torch.arange(n - 3), torch.arange(p.extra_page_count), torch.from_numpy(sc["visible"]))
    with pytest.raises(ValueError, match="Occurrence slots must be int32 or int64"):
        ownership.OccurrenceState.empty(torch.device("cpu"), torch.int16)


def test_empty_state_plans_like_an_unmatched_request(cpu_gather):
    """OccurrenceState.empty equals the state of a request whose match is
    empty, field for field, and plans the same first forward."""
    impl = scenarios.NativeImpl(torch.device("cpu"))
    sc = scenarios.make(7)
    n = sc["n"]
    empty = ownership.OccurrenceState.empty(torch.device("cpu"))
    matched = impl.from_match(np.zeros(0, np.int64), np.zeros(0, np.int32), 0, np.zeros(0, dtype=bool), None)
    for name in ("slots", "owned", "canonical_rows", "terminal_rows", "canonical_positions"):
        a, b = getattr(empty, name), getattr(matched, name)
        assert a.dtype == b.dtype and a.shape == b.shape, name
    assert empty.exact_prefix_len == 0 and empty.swa_resident is None
    win = impl.window(sc["layout"], sc["visible"], 0, n)
    keep = impl.keep(empty, sc["layout"], n)
    pa, pb = impl.plan(empty, win, keep), impl.plan(matched, win, keep)
    for key in ("source_rows", "allocated", "copy_source_rows", "pairs", "terminal_occurrences"):
        assert np.array_equal(pa[key], pb[key]), key


def test_long_lifecycles_match_the_oracle(cpu_gather):
    """Prompts of 300-1500 tokens, up to 12 Drop/Reposition turns and 8
    forwards: the native planner's trace equals the oracle's."""
    native = scenarios.NativeImpl(torch.device("cpu"))
    oracle = scenarios.OracleImpl()
    forwards = 0
    for seed in range(30):
        sc = scenarios.make(5000 + seed, n_range=(300, 1500), max_cuts=8)
        want = scenarios.run(sc, oracle)
        got = scenarios.run(sc, native)
        assert [k for k, _ in got] == [k for k, _ in want], seed
        for (name, a), (_, b) in zip(got, want):
            assert _same(a, b), (seed, name)
        forwards += sum(1 for k, _ in want if k.endswith(".keep"))
    assert forwards > 60


def test_bench_published_terminals_match_the_scheduler_rule(cpu_gather):
    """The benchmark's chunked lifecycle picks each forward's published
    terminal versions with its own helper; it equals the rule of the
    reference scheduler (played by the oracle) at every forward of random
    multi-forward scenarios."""
    import bench

    impl = scenarios.NativeImpl(torch.device("cpu"))
    checked = 0
    for seed in range(12):
        sc = scenarios.make(300 + seed)
        n = sc["n"]
        st = impl.from_match(np.zeros(0, np.int64), np.zeros(0, np.int32), 0, np.zeros(0, dtype=bool), None)
        bounds = sorted({0, n, *[int(b) for b in sc["forwards"] if 0 < b < n]})
        lay = scenarios.torch_layout(sc["layout"])
        for qs, qe in zip(bounds[:-1], bounds[1:]):
            want = impl.keep(st, sc["layout"], qe)
            got = bench._published_terminals(st, lay, qe).numpy()
            assert np.array_equal(got, want), (seed, qs, qe)
            checked += 1
            win = impl.window(sc["layout"], sc["visible"], qs, qe)
            try:
                p = impl.plan(st, win, want)
            except ValueError:
                break
            q = impl._slots(10_000 * (qs + 1) + np.arange(qe - qs))
            extra = impl._slots(900_000 + 10_000 * qs + np.arange(p["extra_page_count"]))
            st, _ = impl.advance(st, win, p, q, extra, sc["visible"])
    assert checked > 20
