"""CPU checks of libakv_amd.so: exports, argument validation, host compiler.

No kernel is launched here; the event compiler is host code.
"""

import re
from pathlib import Path

import numpy as np
import pytest
import torch

from akv_amd import _lib, plan, synth
from oracle import events as oe

HEADER = Path(__file__).resolve().parents[1] / "include" / "akv_amd.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(akv_\w+)\(", text, flags=re.M)))


def test_exports_every_declared_symbol(lib):
    declared = _declared()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.EXPORTED)
    assert lib.akv_version().decode().startswith("akv_amd")


def test_validation_rejects_before_any_device_work(lib):
    rc = lib.akv_reposition_kv_layers(None, None, 1, 7, 8, 64, 64, 512, 64, 512, 64, None, None, None, 2,
                                      1, None, 0, 64, 1, 0, None)
    assert rc == _lib.AKV_EINVAL and "KV dtype" in _lib.last_error()
    rc = lib.akv_reposition_kv_layers(None, None, 1, 2, 8, 64, 63, 512, 64, 512, 64, None, None, None, 2,
                                      1, None, 0, 64, 1, 0, None)
    assert rc == _lib.AKV_EINVAL and "rotary_dim" in _lib.last_error()
    # empty work returns silently, like the reference
    assert lib.akv_reposition_kv_layers(None, None, 0, 2, 8, 64, 64, 512, 64, 512, 64, None, None, None, 2,
                                        0, None, 0, 64, 1, 0, None) == 0
    def zeros(fn, **overrides):
        args = [None if t is _lib.c_void_p else 0 for t in fn.argtypes]
        for i, v in overrides.items():
            args[int(i[1:])] = v
        return args

    assert lib.akv_compact_launches(-1, 0, 0, None) == _lib.AKV_EINVAL
    assert lib.akv_compact_launches(0, 0, 0, None) == 0
    assert lib.akv_compact_rows(*zeros(lib.akv_compact_rows, a0=-1)) == _lib.AKV_EINVAL
    assert lib.akv_compact_rows(*zeros(lib.akv_compact_rows, a0=2)) == _lib.AKV_EINVAL
    assert "null device pointer" in _lib.last_error()
    assert lib.akv_compact_pages(*zeros(lib.akv_compact_pages, a0=-1)) == _lib.AKV_EINVAL
    assert lib.akv_compact_pages(*zeros(lib.akv_compact_pages)) == 0  # empty batch
    assert lib.akv_compact_pages(*zeros(lib.akv_compact_pages, a0=2, a2=5)) == _lib.AKV_EINVAL
    assert "page_size" in _lib.last_error()
    assert lib.akv_compact_pages(*zeros(lib.akv_compact_pages, a0=2, a2=5, a3=16)) == _lib.AKV_EINVAL
    assert "null device pointer" in _lib.last_error()
    assert lib.akv_bind_occurrences(*zeros(lib.akv_bind_occurrences, a0=-1)) == _lib.AKV_EINVAL
    assert lib.akv_bind_occurrences(*zeros(lib.akv_bind_occurrences)) == 0  # empty batch
    assert lib.akv_bind_occurrences(*zeros(lib.akv_bind_occurrences, a0=2, a2=9)) == _lib.AKV_EINVAL
    assert "null device pointer" in _lib.last_error()
    assert lib.akv_bind_workspace_bytes(4, 100000) > 0
    # extend write: n_requests is argument 13
    assert lib.akv_write_extend_rows(*zeros(lib.akv_write_extend_rows, a13=-1)) == _lib.AKV_EINVAL
    assert lib.akv_write_extend_rows(*zeros(lib.akv_write_extend_rows)) == 0  # empty batch
    assert lib.akv_write_extend_rows(*zeros(lib.akv_write_extend_rows, a13=3)) == _lib.AKV_EINVAL
    assert "null device pointer" in _lib.last_error()
    assert lib.akv_context_attention(*zeros(lib.akv_context_attention, a15=1, a17=1, a18=64, a35=4)) == _lib.AKV_EINVAL
    # prefix indices without K/V pools: rejected instead of faulting on the
    # null pool (addresses are never dereferenced on this path)
    fake = 1 << 20
    args = zeros(lib.akv_context_attention, a0=fake, a3=fake, a4=fake, a15=1, a16=8, a17=1, a18=64, a19=fake,
                 a20=fake, a22=fake, a29=0.125, a31=fake, a35=4)
    assert lib.akv_context_attention(*args) == _lib.AKV_EINVAL
    assert "without K/V pools" in _lib.last_error()
    # head dims: multiples of 8 up to 128; at most 128 q heads per KV head;
    # a logit cap is 0 or positive and finite
    for a18, a16, a17, a30, message in [(60, 8, 1, 0.0, "head_dim 60"), (136, 8, 1, 0.0, "head_dim 136"),
                                        (64, 129, 1, 0.0, "at most 128 per KV head"),
                                        (64, 12, 8, 0.0, "at most 128 per KV head"),
                                        (64, 8, 1, -1.0, "logit_cap"), (64, 8, 1, float("inf"), "logit_cap"),
                                        (64, 8, 1, float("nan"), "logit_cap")]:
        bad = zeros(lib.akv_context_attention, a15=1, a16=a16, a17=a17, a18=a18, a29=0.125, a30=a30, a35=4)
        assert lib.akv_context_attention(*bad) == _lib.AKV_EINVAL
        assert message in _lib.last_error(), (message, _lib.last_error())
    assert lib.akv_window_count(*zeros(lib.akv_window_count)) == _lib.AKV_EINVAL
    assert lib.akv_window_compile_bounded(*zeros(lib.akv_window_compile_bounded)) == _lib.AKV_EINVAL
    assert "null host pointer" in _lib.last_error()
    # every pointer present, a negative capacity: rejected before any replay
    one = np.zeros(8, dtype=np.int32)
    caps = np.array([4, 1, -1], dtype=np.int64)
    counts = np.zeros(4, dtype=np.int64)
    p32 = one.ctypes.data
    assert lib.akv_window_compile_bounded(1, p32, p32, p32, 0, p32, p32, p32, p32, p32, 0, 1, caps.ctypes.data,
                                          counts.ctypes.data, *([p32] * 7)) == _lib.AKV_EINVAL
    assert "negative capacity" in _lib.last_error()
    assert lib.akv_decode_attention(*zeros(lib.akv_decode_attention, a9=1, a11=1, a12=64)) == _lib.AKV_EINVAL
    assert "q heads" in _lib.last_error()
    ws = lib.akv_compact_workspace_bytes(64, 65536)
    assert ws > 0
    assert lib.akv_decode_indices(*zeros(lib.akv_decode_indices)) == 0
    assert lib.akv_decode_indices(*zeros(lib.akv_decode_indices, a16=3)) == _lib.AKV_EINVAL
    assert lib.akv_build_indptr(None, 0, 3, None, 0, None, 1, 1, None) == _lib.AKV_EINVAL
    assert lib.akv_gather_slots(*zeros(lib.akv_gather_slots, a0=7)) == _lib.AKV_EINVAL
    assert "slot dtype" in _lib.last_error()
    assert lib.akv_gather_slots(*zeros(lib.akv_gather_slots)) == 0  # nothing to gather
    assert lib.akv_gather_slots(*zeros(lib.akv_gather_slots, a7=5, a8=9)) == _lib.AKV_EINVAL
    assert lib.akv_gather_slots(*zeros(lib.akv_gather_slots, a7=5, a8=5)) == _lib.AKV_EINVAL
    assert "null pointer" in _lib.last_error()
    assert lib.akv_plan_ownership(*zeros(lib.akv_plan_ownership, a0=4, a1=2, a2=1)) == _lib.AKV_EINVAL
    assert "Invalid occurrence ownership/query boundaries" in _lib.last_error()
    assert lib.akv_plan_ownership(*zeros(lib.akv_plan_ownership, a0=4, a1=0, a2=4, a4=4)) == _lib.AKV_EINVAL
    assert "null host pointer" in _lib.last_error()
    assert lib.akv_advance_ownership(*zeros(lib.akv_advance_ownership, a0=4, a1=0, a2=4, a4=3, a12=4)) == _lib.AKV_EINVAL
    assert "Context admission does not cover the selected window" in _lib.last_error()


def _events(n, drops, repos):
    insert = [i for i, _ in drops]
    offsets, flat = [0], []
    for _, ranges in drops:
        for s, e in ranges:
            flat += [s, e]
        offsets.append(offsets[-1] + len(ranges))
    b = torch.tensor(repos, dtype=torch.int32)
    return dict(
        token_ids=torch.arange(n, dtype=torch.int64) * 7 % 1000,
        drop_insert_offsets=torch.tensor(insert, dtype=torch.int32),
        drop_range_offsets=torch.tensor(offsets, dtype=torch.int32),
        drop_ranges=torch.tensor(flat, dtype=torch.int32),
        reposition_raw_boundaries=b,
        reposition_insert_offsets=b + 1,
    )


FIELDS = ["positions", "keep_mask", "birth_positions", "birth_stages", "materialized_stage",
          "transition_offsets", "transition_raw_tokens", "transition_old_positions",
          "transition_new_positions", "effective_reposition_stages", "effective_repositions",
          "ignored_repositions", "drop_event_to_key", "records", "virtual_mask", "key_to_token",
          "token_to_key"]


def _compare(ev):
    got = plan.compile_context_layout(**ev)
    want = oe.compile_context_layout(*(ev[k].numpy() for k in ev))
    for f in FIELDS:
        np.testing.assert_array_equal(getattr(got, f).numpy(), getattr(want, f), err_msg=f)
    assert got.next_position == want.next_position


def test_native_compiler_matches_oracle_on_random_programs():
    rng = np.random.default_rng(7)
    done = 0
    for _ in range(300):
        n = int(rng.integers(1, 90))
        drops = []
        for at in sorted(rng.choice(np.arange(1, n + 1), size=min(n, int(rng.integers(0, 5))), replace=False)):
            cuts = np.sort(rng.choice(np.arange(0, at + 1), size=min(4, at + 1), replace=False))
            ranges = [(int(cuts[i]), int(cuts[i + 1])) for i in range(0, len(cuts) - 1, 2)]
            drops.append((int(at), ranges))
        repos = sorted(rng.choice(np.arange(0, n), size=min(n, int(rng.integers(0, 5))), replace=False).tolist())
        ev = _events(n, drops, repos)
        try:
            oe.compile_context_layout(*(ev[k].numpy() for k in ev))
        except ValueError as err:
            with pytest.raises(ValueError, match=re.escape(str(err))):
                plan.compile_context_layout(**ev)
            continue
        _compare(ev)
        done += 1
    assert done > 150


def test_native_compiler_matches_oracle_on_workloads():
    for name in ("tiny", "gpt-oss-32k"):
        w = synth.workload(name)
        _compare(synth.request_events(w.lengths[0], w.spans[0]))


@pytest.mark.parametrize(
    "kw,message",
    [
        (dict(drop_ranges=torch.tensor([0, 1], dtype=torch.int32)), "drop_range_offsets does not cover drop_ranges"),
        (dict(reposition_insert_offsets=torch.tensor([3], dtype=torch.int32)), "Invalid Reposition event metadata"),
        (dict(token_ids=torch.zeros((2, 2), dtype=torch.int32)), "token_ids must be a one-dimensional CPU integer tensor."),
        (dict(drop_ranges=torch.tensor([2**40, 0], dtype=torch.int64),
              drop_range_offsets=torch.tensor([0, 1], dtype=torch.int32),
              drop_insert_offsets=torch.tensor([5], dtype=torch.int32)), "drop_ranges exceeds the signed int32 range."),
    ],
)
def test_native_compiler_error_messages(kw, message):
    ev = _events(8, [], [5])
    ev.update(kw)
    with pytest.raises(ValueError, match=re.escape(message)):
        plan.compile_context_layout(**ev)
