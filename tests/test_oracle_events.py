"""Pins oracle.events: closed form, an independent brute-force model, the
README block-position example and the reference's runtime invariants."""

import numpy as np
import pytest

from oracle import events as ev


def _compile(n, drops, repositions, tokens=None):
    """drops: list of (insertion, [(start, end), ...]); repositions: raw boundaries."""
    drops = sorted(drops)
    insert = [i for i, _ in drops]
    offsets = [0]
    flat = []
    for _, ranges in drops:
        for s, e in ranges:
            flat += [s, e]
        offsets.append(offsets[-1] + len(ranges))
    tokens = np.arange(n) if tokens is None else tokens
    b = np.asarray(repositions, dtype=np.int64)
    return ev.compile_context_layout(tokens, np.asarray(insert, dtype=np.int64),
                                     np.asarray(offsets, dtype=np.int64),
                                     np.asarray(flat, dtype=np.int64), b, b + 1)


def brute_force(n, drops, repositions):
    """Recompute every position from the active list after each event.

    A Reposition renumbers all active tokens to their rank; the tokens whose
    position changes are its transitions (none -> ignored).  Births take the
    next position.  No linked list, no "first non-compact" bookkeeping.
    """
    drop_at = {i: r for i, r in drops}
    repo_at = {b + 1: b for b in repositions}
    active, pos, next_pos = [], {}, 0
    birth = {}
    trans, stages = [], 0
    for at in range(n + 1):
        if at in drop_at:
            gone = {t for s, e in drop_at[at] for t in range(s, e)}
            active = [t for t in active if t not in gone]
        if at in repo_at:
            if not active:
                raise ValueError("no active")
            changed = [(t, pos[t], r) for r, t in enumerate(active) if pos[t] != r]
            if changed:
                assert all(o > r for _, o, r in changed)
                stages += 1
                trans.append(changed)
                for t, _, r in changed:
                    pos[t] = r
                next_pos = len(active)
        if at < n:
            pos[at] = next_pos
            birth[at] = next_pos
            next_pos += 1
            active.append(at)
    keep = np.zeros(n, dtype=bool)
    keep[active] = True
    return keep, np.array([pos[t] for t in range(n)]), trans, next_pos, stages


def _random_program(rng, n):
    drops = []
    for at in sorted(rng.choice(np.arange(1, n + 1), size=min(n, int(rng.integers(0, 4))), replace=False)):
        k = int(rng.integers(1, 3))
        cuts = np.sort(rng.choice(np.arange(0, at + 1), size=min(2 * k, at + 1), replace=False))
        ranges = [(int(cuts[2 * j]), int(cuts[2 * j + 1])) for j in range(len(cuts) // 2)
                  if cuts[2 * j] < cuts[2 * j + 1]]
        if ranges:
            drops.append((int(at), ranges))
    repos = sorted(rng.choice(np.arange(0, n), size=min(n, int(rng.integers(0, 4))), replace=False).tolist())
    return drops, repos


def test_single_stage_closed_form():
    rng = np.random.default_rng(0)
    for _ in range(50):
        n = int(rng.integers(8, 300))
        k = int(rng.integers(1, 5))
        cuts = np.sort(rng.choice(np.arange(n + 1), size=2 * k, replace=False))
        spans = [(int(cuts[2 * j]), int(cuts[2 * j + 1])) for j in range(k)]
        lay = _compile(n, [(n, spans)], [n - 1])
        keep, pos, moved, old, new, nxt = ev.single_stage_closed_form(n, spans)
        np.testing.assert_array_equal(lay.keep_mask, keep)
        np.testing.assert_array_equal(lay.positions, pos)
        np.testing.assert_array_equal(lay.transition_raw_tokens, moved)
        np.testing.assert_array_equal(lay.transition_old_positions, old)
        np.testing.assert_array_equal(lay.transition_new_positions, new)
        assert lay.next_position == nxt


def test_matches_brute_force_on_random_multi_stage_programs():
    rng = np.random.default_rng(1)
    checked = 0
    for _ in range(400):
        n = int(rng.integers(1, 65))
        drops, repos = _random_program(rng, n)
        try:
            want = brute_force(n, drops, repos)
        except ValueError:
            with pytest.raises(ValueError, match="has no active tokens"):
                _compile(n, drops, repos)
            continue
        lay = _compile(n, drops, repos)
        keep, pos, trans, next_pos, stages = want
        np.testing.assert_array_equal(lay.keep_mask, keep)
        np.testing.assert_array_equal(lay.positions, pos)
        assert lay.next_position == next_pos
        assert len(lay.transition_offsets) == stages + 1
        flat = [x for stage in trans for x in stage]
        np.testing.assert_array_equal(lay.transition_raw_tokens, [t for t, _, _ in flat])
        np.testing.assert_array_equal(lay.transition_old_positions, [o for _, o, _ in flat])
        np.testing.assert_array_equal(lay.transition_new_positions, [r for _, _, r in flat])
        np.testing.assert_array_equal(np.diff(lay.transition_offsets), [len(s) for s in trans])
        # replaying transitions over birth positions reproduces the final positions
        cur = lay.birth_positions.astype(np.int64).copy()
        for a, b in zip(lay.transition_offsets[:-1], lay.transition_offsets[1:]):
            ids = lay.transition_raw_tokens[a:b]
            np.testing.assert_array_equal(cur[ids], lay.transition_old_positions[a:b])
            cur[ids] = lay.transition_new_positions[a:b]
        np.testing.assert_array_equal(cur, lay.positions)
        checked += 1
    assert checked > 200


def test_readme_block_positions():
    # README.md:269-280: blocks A..F, one token each; drops A@3, B@4, C@5, D@6;
    # Reposition at turns 4 and 6
    drops = [(3, [(0, 1)]), (4, [(1, 2)]), (5, [(2, 3)]), (6, [(3, 4)])]
    turn4 = _compile(4, [d for d in drops if d[0] <= 4], [3])
    assert turn4.keep_mask.tolist() == [False, False, True, True]
    assert turn4.positions[2:].tolist() == [0, 1]  # C(0), D(1)
    turn5 = _compile(5, [d for d in drops if d[0] <= 5], [3])
    assert turn5.positions[3:].tolist() == [1, 2]  # D(1), E(2)
    turn6 = _compile(6, drops, [3, 5])
    assert turn6.keep_mask.tolist() == [False] * 4 + [True, True]
    assert turn6.positions[4:].tolist() == [0, 1]  # E(0), F(1)


def test_records_and_keys():
    lay = _compile(6, [(4, [(1, 3)])], [3])
    kinds = lay.records[:, 0].tolist()
    assert kinds == [0, 0, 0, 0, ev.DELTA_KIND, ev.REPOSITION_KIND, 0, 0]
    assert lay.records[4].tolist() == [1, -2, -4]
    assert lay.records[5].tolist() == [2, 3, -1]
    assert lay.token_to_key.tolist() == [0, 1, 2, 3, 6, 7]
    assert lay.virtual_mask.tolist() == [False] * 4 + [True, True] + [False] * 2
    assert lay.drop_event_to_key.tolist() == [4]
    # final positions ride in the token records
    np.testing.assert_array_equal(lay.records[lay.token_to_key, 2], lay.positions)


def test_ignored_reposition_keeps_next_position():
    lay = _compile(8, [(8, [(6, 8)])], [7])
    assert lay.ignored_repositions.tolist() == [True]
    assert lay.next_position == 8
    assert len(lay.transition_raw_tokens) == 0


@pytest.mark.parametrize(
    "drops,repos,message",
    [
        ([(3, [(2, 4)])], [], "Drop ranges must be ordered, disjoint, and already materialized"),
        ([(4, [(2, 3), (1, 2)])], [], "Drop ranges must be ordered, disjoint, and already materialized"),
        ([(9, [(0, 1)])], [], "Invalid Drop event metadata"),
        ([(3, [(0, 3)])], [2], "Reposition at raw boundary 2 has no active tokens."),
    ],
)
def test_errors(drops, repos, message):
    with pytest.raises(ValueError, match=message.replace(".", r"\.")):
        _compile(8, drops, repos)


def test_token_id_range():
    with pytest.raises(ValueError, match="outside the non-negative int32 range"):
        _compile(3, [], [], tokens=np.array([0, -5, 2]))
