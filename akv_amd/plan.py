"""Drop-in ``compile_context_layout`` on the native host event compiler.

Same inputs, outputs (``ContextLayout``), validation and ``ValueError``
messages as ``compile_context_layout``
(``akv/system/sglang/srt/context_system/ir.py:113-274``); the two replay
passes run in ``akv_plan_count`` / ``akv_plan_compile`` of ``libakv_amd.so``
(host C++, no device work) instead of a tvm-ffi JIT module.
"""

import time
from dataclasses import dataclass

import torch

from . import _lib

TOKEN_KIND = 0
DELTA_KIND = 1
REPOSITION_KIND = 2


@dataclass(frozen=True)
class ContextLayout:
    drop_insert_offsets: torch.Tensor
    drop_range_offsets: torch.Tensor
    drop_ranges: torch.Tensor
    records: torch.Tensor
    virtual_mask: torch.Tensor
    key_to_token: torch.Tensor
    token_to_key: torch.Tensor
    positions: torch.Tensor
    keep_mask: torch.Tensor
    materialized_stage: torch.Tensor
    birth_positions: torch.Tensor
    birth_stages: torch.Tensor
    transition_offsets: torch.Tensor
    transition_raw_tokens: torch.Tensor
    transition_old_positions: torch.Tensor
    transition_new_positions: torch.Tensor
    effective_reposition_stages: torch.Tensor
    drop_event_to_key: torch.Tensor
    effective_repositions: torch.Tensor
    ignored_repositions: torch.Tensor
    next_position: int
    compile_ns: int

    @property
    def keys(self) -> torch.Tensor:
        return self.records


def compile_context_layout(
    token_ids: torch.Tensor,
    drop_insert_offsets: torch.Tensor,
    drop_range_offsets: torch.Tensor,
    drop_ranges: torch.Tensor,
    reposition_raw_boundaries: torch.Tensor,
    reposition_insert_offsets: torch.Tensor,
) -> ContextLayout:
    """Compile raw-token events into final positions and Reposition transitions.

    Drop offsets are insertion points (the next query); intervals are
    half-open raw-token ranges.  Reposition boundaries are the preceding raw
    token.  Drop runs before Reposition at a shared insertion point.
    """
    vectors = {
        "token_ids": token_ids,
        "drop_insert_offsets": drop_insert_offsets,
        "drop_range_offsets": drop_range_offsets,
        "drop_ranges": drop_ranges,
        "reposition_raw_boundaries": reposition_raw_boundaries,
        "reposition_insert_offsets": reposition_insert_offsets,
    }
    for name, value in vectors.items():
        if (
            value.device.type != "cpu"
            or value.ndim != 1
            or value.dtype not in (torch.int32, torch.int64)
        ):
            raise ValueError(f"{name} must be a one-dimensional CPU integer tensor.")
        if (
            value.dtype == torch.int64
            and len(value)
            and (int(value.min()) < -(2**31) or int(value.max()) >= 2**31)
        ):
            raise ValueError(f"{name} exceeds the signed int32 range.")
    token_ids = token_ids.contiguous()
    drop_insert_offsets = drop_insert_offsets.to(torch.int32).contiguous()
    drop_range_offsets = drop_range_offsets.to(torch.int32).contiguous()
    drop_ranges = drop_ranges.to(torch.int32).contiguous()
    reposition_raw_boundaries = reposition_raw_boundaries.to(torch.int32).contiguous()
    reposition_insert_offsets = reposition_insert_offsets.to(torch.int32).contiguous()
    if (
        len(drop_range_offsets) != len(drop_insert_offsets) + 1
        or len(drop_ranges) % 2
        or len(reposition_insert_offsets) != len(reposition_raw_boundaries)
    ):
        raise ValueError("Reposition transition-count tensor lengths are inconsistent")

    lib = _lib.load()
    started = time.perf_counter_ns()
    n = len(token_ids)
    repositions = len(reposition_raw_boundaries)
    counts = torch.zeros(repositions, dtype=torch.int32)
    count_status = torch.zeros(2, dtype=torch.int64)
    rc = lib.akv_plan_count(
        n,
        drop_insert_offsets.data_ptr(),
        len(drop_insert_offsets),
        drop_range_offsets.data_ptr(),
        drop_ranges.data_ptr(),
        len(drop_ranges),
        reposition_raw_boundaries.data_ptr(),
        reposition_insert_offsets.data_ptr(),
        repositions,
        counts.data_ptr(),
        count_status.data_ptr(),
    )
    _lib.check(rc, "akv_plan_count")
    if int(count_status[0]) == 1:
        raise ValueError(
            f"Reposition at raw boundary {int(count_status[1])} has no active tokens."
        )
    transitions = int(counts.sum())
    capacity = n + len(drop_ranges) // 2 + repositions
    i32, i64 = torch.int32, torch.int64
    records = torch.empty((capacity, 3), dtype=i32)
    virtual_mask = torch.empty(capacity, dtype=torch.bool)
    key_to_token = torch.empty(capacity, dtype=i64)
    token_to_key = torch.empty(n, dtype=i64)
    positions = torch.empty(n, dtype=i32)
    keep_mask = torch.empty(n, dtype=torch.bool)
    materialized_stage = torch.empty(n, dtype=i32)
    birth_positions = torch.empty(n, dtype=i32)
    birth_stages = torch.empty(n, dtype=i32)
    transition_offsets = torch.empty(repositions + 1, dtype=i32)
    transition_raw_tokens = torch.empty(transitions, dtype=i32)
    transition_old_positions = torch.empty(transitions, dtype=i32)
    transition_new_positions = torch.empty(transitions, dtype=i32)
    effective_stages = torch.full((repositions,), -1, dtype=i32)
    drop_event_to_key = torch.full((len(drop_insert_offsets),), -1, dtype=i64)
    effective = torch.zeros(repositions, dtype=torch.bool)
    ignored = torch.zeros(repositions, dtype=torch.bool)
    status = torch.zeros(5, dtype=i64)
    rc = lib.akv_plan_compile(
        token_ids.data_ptr(),
        _lib.AKV_I64 if token_ids.dtype == torch.int64 else _lib.AKV_I32,
        n,
        drop_insert_offsets.data_ptr(),
        len(drop_insert_offsets),
        drop_range_offsets.data_ptr(),
        drop_ranges.data_ptr(),
        len(drop_ranges),
        reposition_raw_boundaries.data_ptr(),
        reposition_insert_offsets.data_ptr(),
        repositions,
        records.data_ptr(),
        virtual_mask.data_ptr(),
        key_to_token.data_ptr(),
        capacity,
        token_to_key.data_ptr(),
        positions.data_ptr(),
        keep_mask.data_ptr(),
        materialized_stage.data_ptr(),
        birth_positions.data_ptr(),
        birth_stages.data_ptr(),
        transition_offsets.data_ptr(),
        transition_raw_tokens.data_ptr(),
        transition_old_positions.data_ptr(),
        transition_new_positions.data_ptr(),
        transitions,
        effective_stages.data_ptr(),
        drop_event_to_key.data_ptr(),
        effective.data_ptr(),
        ignored.data_ptr(),
        status.data_ptr(),
    )
    _lib.check(rc, "akv_plan_compile")
    if int(status[0]) == 1:
        raise ValueError(f"Reposition at raw boundary {int(status[4])} has no active tokens.")
    if int(status[0]) == 2:
        raise ValueError(
            f"Reposition Radix token ID {int(status[4])} is outside the non-negative int32 range."
        )
    key_len = int(status[1])
    stages = int(status[2])
    return ContextLayout(
        drop_insert_offsets=drop_insert_offsets,
        drop_range_offsets=drop_range_offsets,
        drop_ranges=drop_ranges,
        records=records[:key_len],
        virtual_mask=virtual_mask[:key_len],
        key_to_token=key_to_token[:key_len],
        token_to_key=token_to_key,
        positions=positions,
        keep_mask=keep_mask,
        materialized_stage=materialized_stage,
        birth_positions=birth_positions,
        birth_stages=birth_stages,
        transition_offsets=transition_offsets[: stages + 1],
        transition_raw_tokens=transition_raw_tokens,
        transition_old_positions=transition_old_positions,
        transition_new_positions=transition_new_positions,
        effective_reposition_stages=effective_stages,
        drop_event_to_key=drop_event_to_key,
        effective_repositions=effective,
        ignored_repositions=ignored,
        next_position=int(status[3]),
        compile_ns=time.perf_counter_ns() - started,
    )
