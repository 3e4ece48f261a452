"""Pins oracle.decode against the compacted-row identity and direct counts."""

import numpy as np

from oracle import decode as dec
from oracle import events as ev
from oracle import occurrence as occ


def _request(rng, n, generated):
    k = int(rng.integers(1, 4))
    cuts = np.sort(rng.choice(np.arange(n + 1), size=2 * k, replace=False))
    spans = [(int(cuts[2 * j]), int(cuts[2 * j + 1])) for j in range(k)]
    lay = ev.compile_context_layout(np.arange(n), np.array([n]), np.array([0, k]),
                                    np.array([x for s in spans for x in s]), np.array([n - 1]), np.array([n]))
    if not lay.keep_mask.any():
        return None
    return lay


def _registry(rng, batch, width):
    """A registry/table pair over random requests; returns what the identity needs."""
    table = np.full((batch + 2, width), -1, dtype=np.int32)
    registry = np.zeros((batch + 2, 6), dtype=np.int64)
    memory, expect, lengths, rows = {}, [], [], []
    handle = 1000
    for b in range(batch):
        row = b + 1
        n = int(rng.integers(4, 60))
        gen = int(rng.integers(1, 5))
        lay = _request(rng, n, gen)
        if lay is None or rng.random() < 0.2:
            # ordinary request: plain raw row
            length = n + gen
            table[row, :length] = rng.integers(1, 10**6, size=length)
            expect.append(table[row, :length].copy())
            lengths.append(length)
            rows.append(row)
            continue
        slots = rng.integers(1, 10**6, size=n + gen).astype(np.int32)
        moved = lay.keep_mask & (lay.birth_positions != lay.positions)
        out = occ.closed_form(slots[:n], lay.keep_mask, lay.birth_positions, lay.positions,
                              rng.integers(1, 10**6, size=int(moved.sum())))
        table[row, :n] = out["terminal_row"]
        table[row, n : n + gen] = slots[n:]
        raw, pos = occ.decode_layout(lay)
        memory[handle], memory[handle + 1] = raw, pos
        registry[row] = (handle, handle + 1, n, len(raw), lay.next_position, 0)
        handle += 2
        # request_active_slots: compacted row, then the generated tail
        expect.append(np.concatenate((table[row, raw], table[row, n : n + gen])))
        lengths.append(len(raw) + gen)
        rows.append(row)
    return table, registry, memory, expect, np.array(lengths), np.array(rows)


def test_indices_equal_compacted_rows():
    rng = np.random.default_rng(0)
    table, registry, memory, expect, lengths, rows = _registry(rng, 12, 80)
    indptr = dec.kv_indptr(lengths)
    np.testing.assert_array_equal(indptr[1:], np.cumsum(lengths))
    out = np.full(indptr[-1], -7, dtype=np.int64)
    dec.decode_indices(registry, table, rows, lengths, indptr, out, memory=memory)
    np.testing.assert_array_equal(out, np.concatenate(expect))
    # translation multiplies the mapped slot
    mapping = np.arange(10**6, dtype=np.int64) * 3 + 1
    out2 = np.zeros_like(out)
    dec.decode_indices(registry, table, rows, lengths, indptr, out2, memory=memory, mapping=mapping, multiplier=2)
    np.testing.assert_array_equal(out2, (np.concatenate(expect) * 3 + 1) * 2)


def test_window_lengths_count_visible_keys():
    rng = np.random.default_rng(1)
    table, registry, memory, expect, lengths, rows = _registry(rng, 16, 80)
    for window in (0, 1, 5, 17, 200):
        got = dec.window_lengths(registry, rows, lengths, window, memory=memory)
        for b, row in enumerate(rows):
            pointer, ppos, prompt, active, next_pos, _ = registry[row]
            if pointer == 0:
                assert got[b] == min(lengths[b], window)
                continue
            gen = lengths[b] - active
            q = next_pos + gen - 1
            positions = np.concatenate((memory[ppos], np.arange(next_pos, next_pos + gen)))
            assert got[b] == np.count_nonzero(q - positions <= window)
    # starts + window lengths select the last visible keys of the compacted row
    window = 5
    got = dec.window_lengths(registry, rows, lengths, window, memory=memory)
    starts = lengths - got
    indptr = dec.kv_indptr(got)
    out = np.zeros(indptr[-1], dtype=np.int64)
    dec.decode_indices(registry, table, rows, got, indptr, out, memory=memory, starts=starts)
    for b in range(len(rows)):
        np.testing.assert_array_equal(out[indptr[b] : indptr[b + 1]], expect[b][starts[b]:])


def test_write_row_slots_and_last_page():
    memory = {11: np.zeros(8, dtype=np.int32), 22: np.zeros(8, dtype=np.int32)}
    dec.write_row_slots(np.array([11, 22]), [0, 1, 1], [2, 0, 7], [5, 6, 7], memory=memory)
    assert memory[11].tolist() == [0, 0, 5, 0, 0, 0, 0, 0]
    assert memory[22].tolist() == [6, 0, 0, 0, 0, 0, 0, 7]
    np.testing.assert_array_equal(dec.last_page_lengths([0, 1, 16, 17, 33], 16), [0, 1, 16, 1, 1])
