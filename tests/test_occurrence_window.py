"""Host occurrence-window compiler (C++) against the oracle's restatement,
and the oracle's window against an independent per-query model of what
each query reads."""

import numpy as np
import pytest
import torch

from akv_amd import occurrence as ow
from akv_amd import plan
from oracle import events as ev
from oracle import occurrence as occ


def _program(rng, n):
    """Random multi-stage program: up to 3 (Drop, Reposition) events inside the prompt."""
    k = int(rng.integers(1, 4))
    inserts = np.sort(rng.choice(np.arange(4, n), size=k, replace=False))
    drops, offsets, visible = [], [0], np.full(n, 2**31 - 1, dtype=np.int64)
    lo = 0
    for at in inserts:
        s = int(rng.integers(lo, max(lo + 1, at - 1)))
        e = int(min(at, s + rng.integers(1, 4)))
        if s < e and (not drops or s >= drops[-1]):
            drops += [s, e]
            offsets.append(len(drops) // 2)
            visible[s:e] = np.minimum(visible[s:e], at)
        else:
            offsets.append(offsets[-1])
        lo = at
    keep_events = np.flatnonzero(np.diff(offsets) > 0)
    ins = inserts[keep_events]
    offs = np.concatenate(([0], np.cumsum(np.diff(offsets)[keep_events])))
    events = dict(token_ids=np.arange(n), drop_insert_offsets=ins, drop_range_offsets=offs,
                  drop_ranges=np.array(drops, dtype=np.int64), reposition_raw_boundaries=inserts - 1,
                  reposition_insert_offsets=inserts)
    return events, visible


def _torch_layout(events):
    t = {k: torch.from_numpy(np.asarray(v)).to(torch.int32) for k, v in events.items()}
    return plan.compile_context_layout(**t)


def test_window_matches_oracle_field_for_field():
    rng = np.random.default_rng(7)
    for _ in range(80):
        n = int(rng.integers(8, 120))
        events, visible = _program(rng, n)
        ref = ev.compile_context_layout(*(np.asarray(events[k]) for k in events))
        want = occ.compile_window(ref, visible)
        lay = _torch_layout(events)
        vis = torch.from_numpy(np.minimum(visible, 2**31 - 1).astype(np.int32))
        got = ow.compile_occurrence_window(lay, vis, lay.positions, query_start=0, query_end=n)
        np.testing.assert_array_equal(got.occurrence_raw_tokens.numpy(), want["raw"])
        np.testing.assert_array_equal(got.occurrence_positions.numpy(), want["pos"])
        np.testing.assert_array_equal(got.terminal_occurrences.numpy(), want["terminal"])
        np.testing.assert_array_equal(got.segment_key_occurrences.numpy(), want["keys"])
        offs = got.segment_key_offsets.numpy()
        assert offs[0] == 0 and offs[-1] == len(want["keys"])
        assert got.segment_query_starts[0] == 0 and got.segment_query_ends[-1] == n
        np.testing.assert_array_equal(got.segment_query_starts[1:].numpy(), got.segment_query_ends[:-1].numpy())


def _positions_at(ref, u, stage):
    """Position of raw token u after the transitions of stages 1..stage (brute force)."""
    p = int(ref.birth_positions[u])
    offs = ref.transition_offsets
    for s in range(1, stage + 1):
        for i in range(int(offs[s - 1]), int(offs[s])):
            if int(ref.transition_raw_tokens[i]) == u:
                p = int(ref.transition_new_positions[i])
    return p


def test_each_query_reads_exactly_the_visible_tokens_at_their_current_positions():
    # independent model: query t of stage s reads every u < t still visible at t
    # (visible_until[u] > t) at its position after the transitions of stages <= s,
    # plus its own birth version; the window's segment keys must say the same
    rng = np.random.default_rng(8)
    for _ in range(40):
        n = int(rng.integers(8, 60))
        events, visible = _program(rng, n)
        ref = ev.compile_context_layout(*(np.asarray(events[k]) for k in events))
        w = occ.compile_window(ref, visible)
        lay = _torch_layout(events)
        vis = torch.from_numpy(np.minimum(visible, 2**31 - 1).astype(np.int32))
        got = ow.compile_occurrence_window(lay, vis, lay.positions, query_start=0, query_end=n)
        raw, pos = got.occurrence_raw_tokens.numpy(), got.occurrence_positions.numpy()
        keys, offs = got.segment_key_occurrences.numpy(), got.segment_key_offsets.numpy()
        starts, ends = got.segment_query_starts.numpy(), got.segment_query_ends.numpy()
        for sg in range(len(starts)):
            seg_keys = keys[offs[sg] : offs[sg + 1]]
            for t in range(starts[sg], ends[sg]):
                stage = int(ref.birth_stages[t])
                # the segment's prefix plus its own queries up to t (causal)
                n_prefix = len(seg_keys) - (ends[sg] - starts[sg])
                seen = seg_keys[: n_prefix + (t - starts[sg]) + 1]
                got_pairs = sorted(zip(raw[seen].tolist(), pos[seen].tolist()))
                want_pairs = sorted([(u, _positions_at(ref, u, stage)) for u in range(t) if visible[u] > t]
                                    + [(t, int(ref.birth_positions[t]))])
                assert got_pairs == want_pairs, (sg, t)
        assert w["keys"].tolist() == keys.tolist()


def test_reference_messages():
    lay = _torch_layout(dict(token_ids=np.arange(6), drop_insert_offsets=np.array([4]),
                             drop_range_offsets=np.array([0, 1]), drop_ranges=np.array([1, 2]),
                             reposition_raw_boundaries=np.array([3]), reposition_insert_offsets=np.array([4])))
    vis = torch.full((6,), 2**31 - 1, dtype=torch.int32)
    vis[1] = 4
    with pytest.raises(ValueError, match="outside the raw prompt"):
        ow.compile_occurrence_window(lay, vis, lay.positions, query_start=0, query_end=7)
    with pytest.raises(ValueError, match="must cover the prompt"):
        ow.compile_occurrence_window(lay, vis[:5], lay.positions, query_start=0, query_end=6)
    bad = vis.clone()
    bad[2] = 2
    with pytest.raises(ValueError, match="invisible before it has been computed"):
        ow.compile_occurrence_window(lay, bad, lay.positions, query_start=0, query_end=6)
    with pytest.raises(ValueError, match="disagree with terminal Radix positions"):
        ow.compile_occurrence_window(lay, vis, lay.birth_positions, query_start=0, query_end=6)
    with pytest.raises(ValueError, match="one-dimensional CPU int32"):
        ow.compile_occurrence_window(lay, vis.long(), lay.positions, query_start=0, query_end=6)


@pytest.mark.parametrize("keys_capacity", [None, 1])
def test_single_replay_and_its_fallback_match_the_oracle_on_query_windows(keys_capacity):
    """The one-replay compile (bounded arrays) and, when its key guess is too
    small, the exact second replay give the oracle's window for arbitrary
    query ranges (chunked forwards)."""
    rng = np.random.default_rng(11)
    for _ in range(60):
        n = int(rng.integers(8, 120))
        events, visible = _program(rng, n)
        ref = ev.compile_context_layout(*(np.asarray(events[k]) for k in events))
        qs = int(rng.integers(0, n - 1))
        qe = int(rng.integers(qs + 1, n + 1))
        want = occ.compile_window(ref, visible, query_start=qs, query_end=qe)
        lay = _torch_layout(events)
        vis = torch.from_numpy(np.minimum(visible, 2**31 - 1).astype(np.int32))
        got = ow.compile_occurrence_window(lay, vis, lay.positions, query_start=qs, query_end=qe,
                                           keys_capacity=keys_capacity)
        for field, key in (("occurrence_raw_tokens", "raw"), ("occurrence_positions", "pos"),
                           ("terminal_occurrences", "terminal"), ("segment_key_occurrences", "keys"),
                           ("segment_query_starts", "starts"), ("segment_query_ends", "ends"),
                           ("segment_key_offsets", "key_offsets")):
            np.testing.assert_array_equal(getattr(got, field).numpy(), want[key], err_msg=field)
        assert got.first_final_occurrence <= got.occurrence_count
