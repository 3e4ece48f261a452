"""Seeded request lifecycles for the ownership planner tests.

A scenario is one request: a random multi-stage Drop/Reposition program,
an optional matched prefix borrowed from the cache (some pages evicted,
an exact-prefix boundary, SWA residency), its prompt computed in 1-4
forwards, possibly a resident recovery gap borrowed between two forwards,
then the publication of its terminal versions and a Drop of borrowed raw
tokens.  ``run(scenario, impl)`` drives an implementation through it with
a lowest-first slot allocator that recycles retired slots, and returns a
flat trace of every input and output -- the same trace for every correct
implementation, so traces of the reference module (golden vectors), the
oracle and the native planner compare array for array.
"""

from __future__ import annotations

import numpy as np

from oracle import events as ev

INF = 2**31 - 1
CACHE_BASE = 1_000_000  # cache-owned (borrowed) slots live above this


def _program(rng, n):
    k = int(rng.integers(1, 4 if n < 100 else 12))
    inserts = np.sort(rng.choice(np.arange(3, n), size=min(k, n - 3), replace=False))
    drops, offsets, drop_at = [], [0], []
    visible = np.full(n, INF, dtype=np.int64)
    lo = 0
    for at in inserts:
        if rng.random() < 0.8:
            s = int(rng.integers(lo, max(lo + 1, at - 1)))
            e = int(min(at, s + rng.integers(1, 6)))
            if s < e and (not drops or s >= drops[-1]):
                drops += [s, e]
                visible[s:e] = np.minimum(visible[s:e], at)
                offsets.append(len(drops) // 2)
                drop_at.append(int(at))
        lo = int(at)
    events = dict(
        token_ids=np.arange(n, dtype=np.int64),
        drop_insert_offsets=np.asarray(drop_at, dtype=np.int64),
        drop_range_offsets=np.asarray(offsets, dtype=np.int64),
        drop_ranges=np.asarray(drops, dtype=np.int64),
        reposition_raw_boundaries=(inserts - 1).astype(np.int64),
        reposition_insert_offsets=inserts.astype(np.int64),
    )
    return events, visible


def make(seed, n_range=(10, 90), max_cuts=4):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(*n_range))
    while True:  # redraw programs whose Reposition finds no active token
        events, visible = _program(rng, n)
        try:
            layout = ev.compile_context_layout(*(np.asarray(events[k]) for k in events))
            break
        except ValueError:
            continue
    sc = dict(seed=seed, n=n, layout=layout, visible=np.minimum(visible, INF).astype(np.int32))
    m = int(rng.integers(1, n - 1)) if rng.random() < 0.5 else 0
    cache = CACHE_BASE + rng.permutation(4 * n)
    positions = np.asarray(layout.positions if rng.random() < 0.7 else layout.birth_positions)
    resident = np.ones(n, dtype=bool)
    if rng.random() < 0.3:
        resident[rng.random(n) < 0.1] = False
    swa = rng.random(n) < 0.8 if rng.random() < 0.5 else None
    sc["match"] = dict(slots=cache[:n].astype(np.int64), positions=positions.astype(np.int32), resident=resident,
                       length=m, exact=int(rng.integers(0, m + 1)), swa=swa)
    cuts = sorted(set(int(c) for c in rng.integers(m + 1, n, size=int(rng.integers(0, max_cuts))))) \
        if m + 1 < n else []
    bounds = [m, *[c for c in cuts if m < c < n], n]
    # a recovery gap: the head of one forward's range is borrowed instead
    gap = None
    if rng.random() < 0.4:
        i = int(rng.integers(0, len(bounds) - 1))
        a, b = bounds[i], bounds[i + 1]
        if b - a >= 2:
            gap = (a, int(rng.integers(a + 1, b)))
    sc["forwards"] = bounds
    sc["gap"] = gap
    sc["gap_exact_bump"] = bool(rng.random() < 0.5)
    # chunked prefill publishes every finished chunk to the cache (which may
    # dedup a private page against a cached copy) and drops the borrowed
    # owners no later query needs
    sc["publish_each"] = bool(rng.random() < 0.5)
    # some lifecycles drop borrowed owners of tokens later queries still
    # read (their private terminal copies then become the copy sources)
    sc["drop_needed"] = bool(rng.random() < 0.3)
    sc["publish_replace"] = rng.random(n) < 0.3
    sc["cache_len"] = int(rng.integers(0, n + 1)) if rng.random() < 0.3 else None
    sc["drop"] = rng.random(n) < 0.3
    return sc


class Allocator:
    """Lowest-first allocation over a recycled free set (slot 0 reserved)."""

    def __init__(self):
        self.next = 1
        self.free = []

    def take(self, k):
        self.free.sort()
        got = self.free[:k]
        self.free = self.free[k:]
        while len(got) < k:
            got.append(self.next)
            self.next += 1
        return np.asarray(got, dtype=np.int64)

    def release(self, slots):
        s = [int(x) for x in slots]
        if len(set(s)) != len(s) or set(s) & set(self.free):
            raise AssertionError("a slot was freed twice")
        if any(x >= CACHE_BASE for x in s):
            raise AssertionError("a cache-owned slot was freed by the request")
        self.free += s


def run(sc, impl):
    """Drive ``impl`` through the scenario; returns [(name, array)]."""
    trace = []

    def rec(name, value):
        trace.append((name, None if value is None else np.asarray(value)))

    def record_state(prefix, st):
        for k, v in impl.fields(st).items():
            rec(f"{prefix}.{k}", v)

    layout, visible, n = sc["layout"], sc["visible"], sc["n"]
    mt = sc["match"]
    m = mt["length"]
    alloc = Allocator()

    def publish(prefix, st, length, cache_len, serial):
        """Cache insert: private terminal pages may be deduplicated against
        cached copies (the cache frees the private duplicate)."""
        f = impl.fields(st)
        term = impl.terminal_slots(st)
        rows = f["terminal_rows"]
        dedup = sc["publish_replace"][:length] & (rows >= 0)
        dedup[rows >= 0] &= f["owned"][rows[rows >= 0]]
        if cache_len is not None:
            dedup[cache_len:] = False
        cached = CACHE_BASE + 16 * n + serial * n + np.arange(length, dtype=np.int64)
        matched = np.where(dedup, cached, term)
        swa = None if mt["swa"] is None else sc["publish_replace"][:length] | mt["swa"][:length]
        rec(prefix + ".matched", matched)
        rec(prefix + ".cache_len", np.int64(-1 if cache_len is None else cache_len))
        try:
            st = impl.publish(st, matched, cache_len, swa)
        except ValueError as e:
            rec(prefix + ".error", np.frombuffer(str(e).encode(), dtype=np.uint8))
            return None
        alloc.release(term[dedup])
        record_state(prefix + ".state", st)
        return st

    swa = None if mt["swa"] is None else mt["swa"][:m]
    st = impl.from_match(mt["slots"][:m], mt["positions"][:m], mt["exact"], mt["resident"][:m], swa)
    bounds = sc["forwards"]
    gap = sc["gap"]
    for f, (qs, qe) in enumerate(zip(bounds[:-1], bounds[1:])):
        if gap is not None and qs == gap[0]:
            exact = impl.fields(st)["exact_prefix_len"]
            if sc["gap_exact_bump"]:
                exact = max(exact, gap[1])
            st = impl.gap(st, mt["slots"], mt["positions"], mt["resident"], gap[1], exact,
                          None if mt["swa"] is None else mt["swa"])
            record_state(f"f{f}.gap", st)
            qs = gap[1]
        win = impl.window(layout, visible, qs, qe)
        for k in ("raw", "pos", "terminal", "keys", "starts", "ends", "key_offsets"):
            rec(f"f{f}.window.{k}", win[k])
        keep = impl.keep(st, layout, qe)
        rec(f"f{f}.keep", keep)
        try:
            p = impl.plan(st, win, keep)
        except ValueError as e:
            rec(f"f{f}.error", np.frombuffer(str(e).encode(), dtype=np.uint8))
            return trace
        for k in ("source_rows", "allocated", "copy_source_rows", "pairs", "terminal_occurrences", "read_cached",
                  "repositioned_cached"):
            rec(f"f{f}.plan.{k}", p[k])
        q_slots = alloc.take(qe - qs)
        extra = alloc.take(int(p["extra_page_count"]))
        rec(f"f{f}.query_slots", q_slots)
        rec(f"f{f}.extra_slots", extra)
        st, out = impl.advance(st, win, p, q_slots, extra, visible)
        for k in ("occurrence_slots", "copy_source_slots", "copy_destination_slots", "copy_position_pairs",
                  "retired_slots", "unused_swa_slots", "retired_swa_resident"):
            rec(f"f{f}.adv.{k}", out[k])
        record_state(f"f{f}.state", st)
        alloc.release(out["retired_slots"])  # the forward completed
        if sc["publish_each"] and qe < n:
            st = publish(f"f{f}.pub", st, qe, qe // 2 if sc["drop_needed"] else qe, f)
            if st is None:
                return trace
            keep_mask = np.asarray(layout.keep_mask[:qe], dtype=bool)
            dropped = ~(keep_mask | (visible[:qe] > qe))
            if sc["drop_needed"]:
                dropped |= sc["drop"][:qe]
            st = impl.drop(st, dropped)
            record_state(f"f{f}.drop", st)
    if bounds[-1] != n:
        return trace
    rec("terminal_slots", impl.terminal_slots(st))
    rec("terminal_swa", impl.terminal_swa(st))
    rec("private_slots_before_publish", impl.private(st))
    st = publish("publish", st, n, sc["cache_len"], len(bounds))
    if st is None:
        return trace
    st = impl.drop(st, sc["drop"])
    record_state("drop.state", st)
    rec("private_slots", impl.private(st))
    rec("nonterminal_private_slots", impl.nonterminal(st))
    rec("nonterminal_private_residency", impl.nonterminal_residency(st))
    return trace


def plan_case(seed):
    """Direct call of the plan over arbitrary ownership metadata: random
    presence, ownership, terminal rows, canonical positions and exact-prefix
    boundary, so every branch is taken (including copies from a terminal
    owner when the canonical one is gone, and missing sources)."""
    rng = np.random.default_rng(50_000 + seed)
    sc = make(seed)
    n = sc["n"]
    layout = sc["layout"]
    qs = int(rng.integers(1, n - 1))
    qe = int(rng.integers(qs + 1, n + 1))
    choice = rng.integers(0, 3, size=qs)
    cpos = np.where(choice == 0, layout.birth_positions[:qs],
                    np.where(choice == 1, layout.positions[:qs], rng.integers(0, n, size=qs)))
    present = rng.random(qs) < 0.7
    return dict(sc=sc, qs=qs, qe=qe, canonical_positions=cpos.astype(np.int32),
                canonical_present=present, canonical_owned=rng.random(qs) < 0.5,
                terminal_present=rng.random(qs) < np.where(present, 0.5, 0.95),
                terminal_keep=np.asarray(layout.keep_mask[:qe], dtype=bool) & (rng.random(qe) < 0.9),
                exact=int(rng.integers(0, qs + 1)))


def run_plan_case(case, impl):
    sc = case["sc"]
    win = impl.window(sc["layout"], sc["visible"], case["qs"], case["qe"])
    trace = [("window.raw", win["raw"]), ("window.pos", win["pos"])]
    try:
        p = impl.plan_free(win, case["canonical_positions"], case["canonical_present"], case["canonical_owned"],
                           case["terminal_present"], case["terminal_keep"], case["qs"], case["qe"], case["exact"])
    except ValueError as e:
        return trace + [("error", np.frombuffer(str(e).encode(), dtype=np.uint8))]
    return trace + [(f"plan.{k}", np.asarray(p[k])) for k in (
        "source_rows", "allocated", "copy_source_rows", "pairs", "terminal_occurrences", "read_cached",
        "repositioned_cached")]


class OracleImpl:
    """The oracle restatement behind the scenario interface."""

    def __init__(self):
        from oracle import occurrence as occ
        from oracle import ownership as own

        self.occ, self.own = occ, own

    def window(self, layout, visible, qs, qe):
        return self.occ.compile_window(layout, visible, qs, qe)

    def from_match(self, slots, positions, exact, resident, swa):
        return self.own.State.from_match(slots, positions, exact_prefix_len=exact, resident=resident,
                                         swa_resident=swa)

    def gap(self, st, slots, positions, resident, end, exact, swa):
        return st.reuse_match_gap(slots, positions, resident, end, exact_prefix_len=exact, swa_resident=swa)

    def keep(self, st, layout, qe):
        return st.prefill_terminal_keep(layout, qe)

    def plan(self, st, win, keep):
        return st.plan(win, keep)

    def plan_free(self, win, cpos, present, owned, tpresent, keep, qs, qe, exact):
        return self.own.plan(win, cpos, present, owned, tpresent, keep, query_start=qs, query_end=qe,
                             exact_prefix_len=exact)

    def advance(self, st, win, p, q_slots, extra, visible):
        a = st.advance(win, p, q_slots, extra, visible)
        return a.state, dict(occurrence_slots=a.occurrence_slots, copy_source_slots=a.copy_source_slots,
                             copy_destination_slots=a.copy_destination_slots,
                             copy_position_pairs=a.copy_position_pairs, retired_slots=a.retired_slots,
                             unused_swa_slots=a.unused_swa_slots, retired_swa_resident=a.retired_swa_resident)

    @staticmethod
    def fields(st):
        return dict(slots=st.slots, owned=st.owned, canonical_rows=st.canonical_rows,
                    terminal_rows=st.terminal_rows, canonical_positions=st.canonical_positions,
                    exact_prefix_len=np.int64(st.exact_prefix_len), swa_resident=st.swa_resident)

    def terminal_slots(self, st):
        return st.terminal_slots()

    def terminal_swa(self, st):
        return st.terminal_swa_residency()

    def publish(self, st, matched, cache_len, swa):
        return st.publish(matched, cache_len=cache_len, swa_resident=swa)

    def drop(self, st, mask):
        return st.drop_borrowed_raw(mask)

    def private(self, st):
        return st.private_slots()

    def nonterminal(self, st):
        return st.nonterminal_private_slots()

    def nonterminal_residency(self, st):
        return st.nonterminal_private_residency()


def torch_layout(layout):
    """Oracle layout (numpy) -> the tensor layout the product reads."""
    import torch
    from types import SimpleNamespace

    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32))
    return SimpleNamespace(
        birth_positions=i32(layout.birth_positions), birth_stages=i32(layout.birth_stages),
        transition_offsets=i32(layout.transition_offsets), transition_raw_tokens=i32(layout.transition_raw_tokens),
        transition_old_positions=i32(layout.transition_old_positions),
        transition_new_positions=i32(layout.transition_new_positions), positions=i32(layout.positions),
        keep_mask=torch.from_numpy(np.asarray(layout.keep_mask, dtype=bool).copy()),
        next_position=int(layout.next_position))


class NativeImpl:
    """``akv_amd.ownership`` (C++ host planner + device gathers) behind the
    scenario interface; slots live on ``device`` as ``slot_dtype``.

    The window, the plan, the advance (bind) and the terminal slots run
    natively.  The radix-cache bookkeeping around them -- matches, borrowed
    gaps, the choice of published terminal versions, publication, Drop of
    borrowed owners, private-page and SWA queries -- is the reference
    scheduler's and is not part of the product; here it is played by the
    oracle's ``State`` (pinned by the same golden traces) on host copies of
    the native state's fields."""

    def __init__(self, device, slot_dtype=None):
        import torch

        from akv_amd import occurrence, ownership
        from oracle import ownership as oracle_ownership

        self.torch, self.occ, self.own = torch, occurrence, ownership
        self.oracle = oracle_ownership
        self.device = device
        self.dtype = slot_dtype or torch.int64
        self._layouts = {}

    def _to_oracle(self, st):
        n = self._n
        return self.oracle.State(n(st.slots).astype(np.int64), n(st.owned).copy(), n(st.canonical_rows).copy(),
                                 n(st.terminal_rows).copy(), n(st.canonical_positions).copy(),
                                 int(st.exact_prefix_len), None if st.swa_resident is None else n(st.swa_resident).copy())

    def _from_oracle(self, ost):
        t = self.torch
        return self.own.OccurrenceState(
            self._slots(ost.slots), t.from_numpy(np.asarray(ost.owned, dtype=bool).copy()),
            t.from_numpy(np.asarray(ost.canonical_rows, dtype=np.int64).copy()),
            t.from_numpy(np.asarray(ost.terminal_rows, dtype=np.int64).copy()),
            t.from_numpy(np.asarray(ost.canonical_positions, dtype=np.int32).copy()), int(ost.exact_prefix_len),
            None if ost.swa_resident is None else t.from_numpy(np.asarray(ost.swa_resident, dtype=bool).copy()))

    def _t(self, a, dtype=None, device=None):
        t = self.torch.from_numpy(np.ascontiguousarray(a).copy())
        return t.to(dtype or t.dtype).to(device) if device is not None else t.to(dtype or t.dtype)

    def _slots(self, a):
        return self._t(np.asarray(a, dtype=np.int64), self.dtype, self.device)

    def _bool(self, a):
        return None if a is None else self._t(np.asarray(a, dtype=bool))

    def _layout(self, layout):
        if id(layout) not in self._layouts:
            self._layouts[id(layout)] = (layout, torch_layout(layout))
        return self._layouts[id(layout)][1]

    @staticmethod
    def _n(t):
        return None if t is None else t.detach().cpu().numpy()

    def window(self, layout, visible, qs, qe):
        lay = self._layout(layout)
        w = self.occ.compile_occurrence_window(lay, self._t(visible, self.torch.int32), lay.positions,
                                               query_start=int(qs), query_end=int(qe))
        return dict(raw=w.occurrence_raw_tokens.numpy(), pos=w.occurrence_positions.numpy(),
                    birth=w.birth_occurrences.numpy(), terminal=w.terminal_occurrences.numpy(),
                    keys=w.segment_key_occurrences.numpy(), starts=w.segment_query_starts.numpy(),
                    ends=w.segment_query_ends.numpy(), key_offsets=w.segment_key_offsets.numpy(), _obj=w)

    def from_match(self, slots, positions, exact, resident, swa):
        return self._from_oracle(self.oracle.State.from_match(slots, positions, exact_prefix_len=exact,
                                                              resident=resident, swa_resident=swa))

    def gap(self, st, slots, positions, resident, end, exact, swa):
        return self._from_oracle(self._to_oracle(st).reuse_match_gap(
            slots, positions, resident, end, exact_prefix_len=exact, swa_resident=swa))

    def keep(self, st, layout, qe):
        return self._to_oracle(st).prefill_terminal_keep(layout, qe)

    @staticmethod
    def _plan_dict(p):
        return dict(source_rows=p.source_rows.numpy(), allocated=p.allocated_occurrences.numpy(),
                    copy_source_rows=p.copy_source_rows.numpy(), pairs=p.copy_position_pairs.numpy(),
                    terminal_occurrences=p.terminal_occurrences.numpy(), read_cached=p.read_cached.numpy(),
                    repositioned_cached=p.repositioned_cached.numpy(), extra_page_count=p.extra_page_count, _obj=p)

    def plan(self, st, win, keep):
        return self._plan_dict(st.plan(win["_obj"], self._bool(keep)))

    def plan_free(self, win, cpos, present, owned, tpresent, keep, qs, qe, exact):
        return self._plan_dict(self.own.plan_occurrence_materialization(
            win["_obj"], self._t(cpos, self.torch.int32), self._bool(present), self._bool(owned),
            self._bool(tpresent), self._bool(keep), query_start=int(qs), query_end=int(qe),
            exact_prefix_len=int(exact)))

    def advance(self, st, win, p, q_slots, extra, visible):
        a = st.advance(win["_obj"], p["_obj"], self._slots(q_slots), self._slots(extra),
                       self._t(visible, self.torch.int32))
        n = self._n
        return a.state, dict(occurrence_slots=n(a.occurrence_slots), copy_source_slots=n(a.copy_source_slots),
                             copy_destination_slots=n(a.copy_destination_slots),
                             copy_position_pairs=n(a.copy_position_pairs), retired_slots=n(a.retired_slots),
                             unused_swa_slots=n(a.unused_swa_slots), retired_swa_resident=n(a.retired_swa_resident))

    def fields(self, st):
        n = self._n
        return dict(slots=n(st.slots), owned=n(st.owned), canonical_rows=n(st.canonical_rows),
                    terminal_rows=n(st.terminal_rows), canonical_positions=n(st.canonical_positions),
                    exact_prefix_len=np.int64(st.exact_prefix_len), swa_resident=n(st.swa_resident))

    def terminal_slots(self, st):
        return self._n(st.terminal_slots())

    def terminal_swa(self, st):
        return self._to_oracle(st).terminal_swa_residency()

    def publish(self, st, matched, cache_len, swa):
        return self._from_oracle(self._to_oracle(st).publish(matched, cache_len=cache_len, swa_resident=swa))

    def drop(self, st, mask):
        return self._from_oracle(self._to_oracle(st).drop_borrowed_raw(mask))

    def private(self, st):
        return self._to_oracle(st).private_slots()

    def nonterminal(self, st):
        return self._to_oracle(st).nonterminal_private_slots()

    def nonterminal_residency(self, st):
        return self._to_oracle(st).nonterminal_private_residency()
