"""Pins oracle.occurrence: the restated planner equals the closed form on
single-stage programs and keeps slot conservation on multi-stage ones."""

import numpy as np

from oracle import events as ev
from oracle import occurrence as occ


def _single_stage(rng, n):
    k = int(rng.integers(1, 5))
    cuts = np.sort(rng.choice(np.arange(n + 1), size=2 * k, replace=False))
    spans = [(int(cuts[2 * j]), int(cuts[2 * j + 1])) for j in range(k)]
    flat = [x for s in spans for x in s]
    lay = ev.compile_context_layout(np.arange(n), np.array([n]), np.array([0, k]), np.array(flat),
                                    np.array([n - 1]), np.array([n]))
    visible = np.full(n, 2**31 - 1, dtype=np.int64)
    for s, e in spans:
        visible[s:e] = n
    return lay, visible


def test_planner_equals_closed_form_single_stage():
    rng = np.random.default_rng(0)
    for _ in range(60):
        n = int(rng.integers(8, 400))
        lay, visible = _single_stage(rng, n)
        plan = occ.plan_final_forward(lay, visible)
        slots = rng.permutation(np.arange(1, 4 * n))
        birth_row = slots[:n]
        fresh = slots[n : n + plan["extra_page_count"]]
        got = occ.advance_final_forward(lay, plan, birth_row, fresh)
        want = occ.closed_form(birth_row, lay.keep_mask, lay.birth_positions, lay.positions, fresh)
        for key in ("terminal_row", "retired_slots", "copy_source_slots", "copy_destination_slots",
                    "copy_position_pairs"):
            np.testing.assert_array_equal(got[key], want[key], err_msg=key)
        # M = number of transitions of the single Reposition
        assert plan["extra_page_count"] == len(lay.transition_raw_tokens)


def test_conservation_invariants():
    rng = np.random.default_rng(1)
    for _ in range(40):
        n = int(rng.integers(8, 400))
        lay, _ = _single_stage(rng, n)
        moved = lay.keep_mask & (lay.birth_positions != lay.positions)
        slots = rng.permutation(np.arange(1, 4 * n))
        birth_row, fresh = slots[:n], slots[n : n + int(moved.sum())]
        out = occ.closed_form(birth_row, lay.keep_mask, lay.birth_positions, lay.positions, fresh)
        row = out["terminal_row"]
        live = row[row >= 0]
        assert len(np.unique(live)) == len(live)
        assert len(out["retired_slots"]) == n - int(lay.keep_mask.sum()) + int(moved.sum())
        np.testing.assert_array_equal(
            np.sort(np.concatenate((out["retired_slots"], live))), np.sort(np.concatenate((birth_row, fresh)))
        )
        raw, pos = occ.decode_layout(lay)
        np.testing.assert_array_equal(out["raw_indices"], raw)
        np.testing.assert_array_equal(out["active_positions"], pos)
        np.testing.assert_array_equal(pos, np.arange(len(pos)))  # compact after the Reposition


def test_multi_stage_planner_conserves_slots():
    rng = np.random.default_rng(2)
    for _ in range(40):
        n = int(rng.integers(16, 80))
        a = int(rng.integers(4, n // 2))
        b = int(rng.integers(a + 4, n))
        # drop [1, 3) at insertion a with a Reposition there, then drop [a, a+2) at b with one at b
        drops_at = np.array([a, b])
        ranges = np.array([1, 3, a, a + 2])
        lay = ev.compile_context_layout(np.arange(n), drops_at, np.array([0, 1, 2]), ranges,
                                        np.array([a - 1, b - 1]), np.array([a, b]))
        visible = np.full(n, 2**31 - 1, dtype=np.int64)
        visible[1:3] = a
        visible[a : a + 2] = b
        plan = occ.plan_final_forward(lay, visible)
        slots = rng.permutation(np.arange(1, 6 * n))
        birth_row = slots[:n]
        fresh = slots[n : n + plan["extra_page_count"]]
        out = occ.advance_final_forward(lay, plan, birth_row, fresh)
        row = out["terminal_row"]
        live = row[row >= 0]
        assert len(np.unique(live)) == len(live)
        np.testing.assert_array_equal(
            np.sort(np.concatenate((out["retired_slots"], live))), np.sort(np.concatenate((birth_row, fresh)))
        )
        # every copy reads a birth slot and carries (birth position, occurrence position)
        src = out["copy_source_slots"]
        where = {int(s): i for i, s in enumerate(birth_row)}
        for s, (old, new) in zip(src, out["copy_position_pairs"]):
            assert lay.birth_positions[where[int(s)]] == old and old != new
        # kept tokens whose final position equals the birth one keep their birth slot
        same = lay.keep_mask & (lay.birth_positions == lay.positions)
        np.testing.assert_array_equal(row[same], birth_row[same])
