"""Write ``tests/golden/ownership_vectors.npz``: traces of the reference
module ``akv/system/sglang/srt/context_system/occurrence.py`` over the seeded
request lifecycles of ``tests/ownership_scenarios.py``.

The module is imported by file path from the reference checkout (its only
runtime imports are numpy and torch); nothing of it is copied.  Only the
recorded inputs and outputs are committed.  Run from the repository root in
a container that holds the reference::

    python tests/golden/make_ownership_vectors.py [/path/to/reference]
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import ownership_scenarios as scenarios  # noqa: E402
from golden.ownership_vectors import OUT, PLAN_CASES, SEEDS, pack  # noqa: E402


def _load(reference_root):
    path = Path(reference_root) / "akv/system/sglang/srt/context_system/occurrence.py"
    spec = importlib.util.spec_from_file_location("reference_occurrence", path)
    module = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = module  # dataclasses resolve annotations through it
    spec.loader.exec_module(module)
    return module


def _np(t):
    return None if t is None else t.numpy().copy()


class ReferenceImpl:
    def __init__(self, module):
        self.m = module
        self._layouts = {}

    def _layout(self, layout):
        key = id(layout)
        if key not in self._layouts:
            i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32))
            self._layouts[key] = (layout, SimpleNamespace(
                birth_positions=i32(layout.birth_positions),
                birth_stages=i32(layout.birth_stages),
                transition_offsets=i32(layout.transition_offsets),
                transition_raw_tokens=i32(layout.transition_raw_tokens),
                transition_old_positions=i32(layout.transition_old_positions),
                transition_new_positions=i32(layout.transition_new_positions),
                positions=i32(layout.positions),
                keep_mask=torch.from_numpy(np.asarray(layout.keep_mask, dtype=bool).copy()),
                next_position=int(layout.next_position),
            ))
        return self._layouts[key][1]

    def window(self, layout, visible, qs, qe):
        lay = self._layout(layout)
        w = self.m.compile_occurrence_window(lay, torch.from_numpy(visible.astype(np.int32)), lay.positions,
                                             query_start=int(qs), query_end=int(qe))
        return dict(raw=_np(w.occurrence_raw_tokens), pos=_np(w.occurrence_positions),
                    birth=_np(w.birth_occurrences), terminal=_np(w.terminal_occurrences),
                    keys=_np(w.segment_key_occurrences), starts=_np(w.segment_query_starts),
                    ends=_np(w.segment_query_ends), key_offsets=_np(w.segment_key_offsets), _obj=w)

    def from_match(self, slots, positions, exact, resident, swa):
        return self.m.OccurrenceState.from_match(
            torch.from_numpy(np.asarray(slots, dtype=np.int64).copy()),
            torch.from_numpy(np.asarray(positions, dtype=np.int32).copy()), exact_prefix_len=int(exact),
            resident=torch.from_numpy(np.asarray(resident, dtype=bool).copy()),
            swa_resident=None if swa is None else torch.from_numpy(np.asarray(swa, dtype=bool).copy()))

    def gap(self, st, slots, positions, resident, end, exact, swa):
        return st.reuse_match_gap(
            torch.from_numpy(np.asarray(slots, dtype=np.int64).copy()),
            torch.from_numpy(np.asarray(positions, dtype=np.int32).copy()),
            torch.from_numpy(np.asarray(resident, dtype=bool).copy()), int(end), exact_prefix_len=int(exact),
            swa_resident=None if swa is None else torch.from_numpy(np.asarray(swa, dtype=bool).copy()))

    def keep(self, st, layout, qe):
        return _np(st.prefill_terminal_keep(self._layout(layout), int(qe)))

    def plan(self, st, win, keep):
        p = st.plan(win["_obj"], torch.from_numpy(np.asarray(keep, dtype=bool).copy()))
        return dict(source_rows=_np(p.source_rows), allocated=_np(p.allocated_occurrences),
                    copy_source_rows=_np(p.copy_source_rows), pairs=_np(p.copy_position_pairs),
                    terminal_occurrences=_np(p.terminal_occurrences), read_cached=_np(p.read_cached),
                    repositioned_cached=_np(p.repositioned_cached), extra_page_count=p.extra_page_count, _obj=p)

    def plan_free(self, win, cpos, present, owned, tpresent, keep, qs, qe, exact):
        b = lambda a: torch.from_numpy(np.asarray(a, dtype=bool).copy())
        p = self.m.plan_occurrence_materialization(
            win["_obj"], torch.from_numpy(np.asarray(cpos, dtype=np.int32).copy()), b(present), b(owned),
            b(tpresent), b(keep), query_start=int(qs), query_end=int(qe), exact_prefix_len=int(exact))
        return dict(source_rows=_np(p.source_rows), allocated=_np(p.allocated_occurrences),
                    copy_source_rows=_np(p.copy_source_rows), pairs=_np(p.copy_position_pairs),
                    terminal_occurrences=_np(p.terminal_occurrences), read_cached=_np(p.read_cached),
                    repositioned_cached=_np(p.repositioned_cached))

    def advance(self, st, win, p, q_slots, extra, visible):
        a = st.advance(win["_obj"], p["_obj"], torch.from_numpy(q_slots.copy()), torch.from_numpy(extra.copy()),
                       torch.from_numpy(visible.astype(np.int32)))
        return a.state, dict(occurrence_slots=_np(a.occurrence_slots), copy_source_slots=_np(a.copy_source_slots),
                             copy_destination_slots=_np(a.copy_destination_slots),
                             copy_position_pairs=_np(a.copy_position_pairs), retired_slots=_np(a.retired_slots),
                             unused_swa_slots=_np(a.unused_swa_slots),
                             retired_swa_resident=_np(a.retired_swa_resident))

    @staticmethod
    def fields(st):
        return dict(slots=_np(st.slots), owned=_np(st.owned), canonical_rows=_np(st.canonical_rows),
                    terminal_rows=_np(st.terminal_rows), canonical_positions=_np(st.canonical_positions),
                    exact_prefix_len=np.int64(st.exact_prefix_len), swa_resident=_np(st.swa_resident))

    def terminal_slots(self, st):
        return _np(st.terminal_slots())

    def terminal_swa(self, st):
        return _np(st.terminal_swa_residency())

    def publish(self, st, matched, cache_len, swa):
        return st.publish(torch.from_numpy(np.asarray(matched, dtype=np.int64).copy()), cache_len=cache_len,
                          swa_resident=None if swa is None else torch.from_numpy(np.asarray(swa, dtype=bool).copy()))

    def drop(self, st, mask):
        return st.drop_borrowed_raw(torch.from_numpy(np.asarray(mask, dtype=bool).copy()))

    def private(self, st):
        return _np(st.private_slots())

    def nonterminal(self, st):
        return _np(st.nonterminal_private_slots())

    def nonterminal_residency(self, st):
        return _np(st.nonterminal_private_residency())


def main():
    module = _load(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    impl = ReferenceImpl(module)
    traces = {seed: scenarios.run(scenarios.make(seed), impl) for seed in SEEDS}
    # direct plan calls over arbitrary ownership metadata, keyed 100000 + seed
    for seed in SEEDS:
        traces[PLAN_CASES + seed] = scenarios.run_plan_case(scenarios.plan_case(seed), impl)
    np.savez_compressed(OUT, **pack(traces))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(traces)} scenarios)")


if __name__ == "__main__":
    main()
