"""Pins of the ownership oracle (``oracle/ownership.py``).

1. Golden vectors: traces of the reference module over 200 seeded request
   lifecycles (``tests/golden/ownership_vectors.npz``, written by
   ``tests/golden/make_ownership_vectors.py``) equal the oracle's traces.
2. Symbolic execution, independent of both: every slot of the KV pool holds
   a ``(raw token, position)`` version tag.  Each forward writes its queries'
   birth tags, then its copies move tags (the source must hold the copy's
   raw token at the pair's old position), then every segment key must find
   exactly its occurrence's tag; between forwards every canonical and
   terminal owner row must hold its version, retired pages must be private
   and unreferenced, and over the whole request every private page is either
   retired once or still owned.  The allocator recycles retired slots lowest
   first, so a stale reference reads a wrong tag.
3. At ``query_start = 0`` with nothing borrowed the plan and advance equal
   the whole-prompt restatement of ``oracle/occurrence.py`` (itself pinned
   by a closed form).
"""

from collections import Counter

import numpy as np
import pytest

import ownership_scenarios as scenarios
from golden import ownership_vectors as vectors
from oracle import events as ev
from oracle import occurrence as occ
from oracle import ownership as own

GOLDEN = vectors.OUT


def _same(a, b):
    if a is None or b is None:
        return a is None and b is None
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.astype(np.int64), b.astype(np.int64))


def test_oracle_traces_equal_reference_traces():
    golden = vectors.unpack(np.load(GOLDEN))
    assert len(golden) == 2 * len(vectors.SEEDS)
    errors = 0
    for seed, want in golden.items():
        if seed >= vectors.PLAN_CASES:
            continue
        got = scenarios.run(scenarios.make(seed), scenarios.OracleImpl())
        assert [k for k, _ in got] == [k for k, _ in want], seed
        for (name, a), (_, b) in zip(got, want):
            assert _same(a, b), (seed, name)
        errors += any(k.endswith(".error") for k, _ in want)
    # the set covers both outcomes of a plan over evicted prefix pages
    assert 0 < errors < 60


def test_oracle_plan_equals_reference_plan_on_arbitrary_ownership():
    golden = vectors.unpack(np.load(GOLDEN))
    from_terminal = errors = 0
    for seed in vectors.SEEDS:
        want = golden[vectors.PLAN_CASES + seed]
        case = scenarios.plan_case(seed)
        got = scenarios.run_plan_case(case, scenarios.OracleImpl())
        assert [k for k, _ in got] == [k for k, _ in want], seed
        for (name, a), (_, b) in zip(got, want):
            assert _same(a, b), (seed, name)
        d = dict(want)
        if "error" in d:
            errors += 1
        else:
            from_terminal += int((d["plan.copy_source_rows"] >= case["sc"]["n"]).sum())
    assert from_terminal > 20 and 20 < errors < 180


def _symbolic(sc, trace):
    """Symbolic execution of the KV pool over one traced lifecycle; returns
    the number of forwards checked, or None when the lifecycle stopped."""
    t = dict(trace)
    seed = sc["seed"]
    layout, n, visible = sc["layout"], sc["n"], sc["visible"]
    birth_pos = np.asarray(layout.birth_positions)
    final_pos = np.asarray(layout.positions)
    mt = sc["match"]
    pool, swa_ok = {}, {}
    for r in range(n):
        if mt["resident"][r]:
            pool[int(mt["slots"][r])] = (r, int(mt["positions"][r]))
        swa_ok[int(mt["slots"][r])] = True if mt["swa"] is None else bool(mt["swa"][r])
    private = Counter()  # pages the request owns

    def check_state(prefix):
        slots, owned = t[prefix + ".slots"], t[prefix + ".owned"]
        cr, tr, cpos = t[prefix + ".canonical_rows"], t[prefix + ".terminal_rows"], t[prefix + ".canonical_positions"]
        for r in range(len(cr)):
            if cr[r] >= 0:
                assert pool.get(int(slots[cr[r]])) == (r, int(cpos[r])), (seed, prefix, r)
            if tr[r] >= 0:
                assert pool.get(int(slots[tr[r]])) == (r, int(final_pos[r])), (seed, prefix, r)
        assert Counter(slots[owned].tolist()) == private, (seed, prefix)
        if t[prefix + ".swa_resident"] is not None:
            assert t[prefix + ".swa_resident"].tolist() == [swa_ok.get(int(x)) for x in slots.tolist()], (seed, prefix)

    def publish(prefix, before):
        if prefix + ".error" in t:
            return False
        slots, owned, tr = t[before + ".slots"], t[before + ".owned"], t[before + ".terminal_rows"]
        matched, cache_len = t[prefix + ".matched"], int(t[prefix + ".cache_len"])
        length = len(tr) if cache_len < 0 else cache_len
        pub_swa = None if mt["swa"] is None else sc["publish_replace"] | mt["swa"]
        for r in range(length):
            if tr[r] < 0:
                continue
            old, new = int(slots[tr[r]]), int(matched[r])
            if owned[tr[r]]:
                private[old] -= 1  # handed to the cache
            if new != old:  # the cache kept its own copy of the same version
                pool[new] = pool[old]
                pool[old] = None
            swa_ok[new] = True if pub_swa is None else bool(pub_swa[r])
        check_state(prefix + ".state")
        return True

    f = 0
    last = None
    while f"f{f}.keep" in t:
        p = f"f{f}."
        if p + "gap.slots" in t:
            check_state(p + "gap")
        if p + "error" in t:
            # a plan may only fail when a borrowed page was evicted or dropped
            assert sc["drop_needed"] or not mt["resident"].all(), seed
            return None
        raw, pos = t[p + "window.raw"], t[p + "window.pos"]
        qs, qe = int(t[p + "window.starts"][0]), int(t[p + "window.ends"][-1])
        q_slots, extra = t[p + "query_slots"], t[p + "extra_slots"]
        private.update(q_slots.tolist() + extra.tolist())
        for i, r in enumerate(range(qs, qe)):
            pool[int(q_slots[i])] = (r, int(birth_pos[r]))
            swa_ok[int(q_slots[i])] = True
        for s in extra.tolist():
            pool[s] = None
            swa_ok[s] = True
        writes = []
        fresh = set(extra.tolist())
        for j, o in enumerate(t[p + "plan.allocated"].tolist()):
            src, dst = int(t[p + "adv.copy_source_slots"][j]), int(t[p + "adv.copy_destination_slots"][j])
            old, new = t[p + "adv.copy_position_pairs"][j].tolist()
            assert dst in fresh and pool.get(src) == (int(raw[o]), old) and new == int(pos[o]), (seed, f, j)
            writes.append((dst, (int(raw[o]), new), swa_ok[src]))
        for dst, tag, ok in writes:
            pool[dst] = tag
            swa_ok[dst] = ok
        if t[p + "adv.unused_swa_slots"] is not None:
            assert t[p + "adv.unused_swa_slots"].tolist() == [d for d, _, ok in writes if not ok]
        occ_slots = t[p + "adv.occurrence_slots"]
        for o in np.unique(t[p + "window.keys"]).tolist():
            assert pool.get(int(occ_slots[o])) == (int(raw[o]), int(pos[o])), (seed, f, o)
        retired = t[p + "adv.retired_slots"].tolist()
        if t[p + "adv.retired_swa_resident"] is not None:
            assert t[p + "adv.retired_swa_resident"].tolist() == [swa_ok[s] for s in retired]
        for s in retired:
            assert private[s] > 0, (seed, f, s)  # only private pages retire
            private[s] -= 1
            pool[s] = None
        check_state(p + "state")
        last = p + "state"
        if p + "pub.matched" in t:
            if not publish(p + "pub", last):
                return None
            check_state(p + "drop")
            last = p + "drop"
        f += 1
    if "terminal_slots" not in t:
        return None
    term = t["terminal_slots"]
    for r in range(n):
        if term[r] >= 0:
            assert pool.get(int(term[r])) == (r, int(final_pos[r])), (seed, r)
        elif layout.keep_mask[r]:
            assert not mt["resident"][r], (seed, r)  # only an evicted borrowed page leaves a hole
    if not publish("publish", last):
        return None
    check_state("drop.state")
    return f


def test_symbolic_execution_of_random_lifecycles():
    forwards = completed = 0
    for seed in range(400):
        sc = scenarios.make(seed)
        done = _symbolic(sc, scenarios.run(sc, scenarios.OracleImpl()))
        if done is not None:
            forwards += done
            completed += 1
    assert completed > 300 and forwards > completed


def test_fresh_request_reduces_to_the_whole_prompt_planner():
    rng = np.random.default_rng(11)
    for seed in range(60):
        sc = scenarios.make(1000 + seed)
        layout, visible, n = sc["layout"], sc["visible"], sc["n"]
        win = occ.compile_window(layout, visible)
        st = own.State.from_match(np.zeros(0, np.int64), np.zeros(0, np.int32), exact_prefix_len=0)
        keep = st.prefill_terminal_keep(layout, n)
        np.testing.assert_array_equal(keep, layout.keep_mask)
        p = st.plan(win, keep)
        ref = occ.plan_final_forward(layout, visible)
        np.testing.assert_array_equal(p["source_rows"], ref["source_rows"])
        np.testing.assert_array_equal(p["allocated"], ref["allocated"])
        np.testing.assert_array_equal(p["pairs"], ref["pairs"])
        q = rng.permutation(np.arange(1, 10 * n))[:n]
        extra = np.arange(10 * n, 10 * n + p["extra_page_count"])
        a = st.advance(win, p, q, extra, visible)
        b = occ.advance_final_forward(layout, ref, q, extra)
        np.testing.assert_array_equal(a.occurrence_slots, b["occurrence_slots"])
        np.testing.assert_array_equal(a.copy_source_slots, b["copy_source_slots"])
        np.testing.assert_array_equal(a.copy_destination_slots, b["copy_destination_slots"])
        np.testing.assert_array_equal(a.retired_slots, b["retired_slots"])
        np.testing.assert_array_equal(a.state.terminal_slots(), b["terminal_row"])


def test_plan_messages():
    layout = ev.compile_context_layout(np.arange(6), np.array([4]), np.array([0, 1]), np.array([1, 2]),
                                       np.array([3]), np.array([4]))
    vis = np.full(6, 2**31 - 1, dtype=np.int64)
    vis[1] = 4
    win = occ.compile_window(layout, vis, 2, 6)
    z = np.zeros(2, dtype=bool)
    with pytest.raises(ValueError, match="Invalid occurrence ownership/query boundaries"):
        own.plan(win, np.zeros(2, np.int32), z, z, z, np.ones(6, bool), query_start=2, query_end=6,
                 exact_prefix_len=3)
    # token 0 is read by every later query but its borrowed page is gone
    with pytest.raises(ValueError, match=r"Occurrence recovery required for raw tokens \[0"):
        own.plan(win, np.asarray(layout.positions[:2], np.int32), np.array([False, True]), z, z,
                 np.ones(6, bool), query_start=2, query_end=6, exact_prefix_len=0)
