"""Host side of the prefill context attention: plan packing and the
reference's validation messages (no kernel launch)."""

import numpy as np
import pytest
import torch

from akv_amd import context_attention as ca


def test_merge_packs_fields_and_offsets_occurrences():
    seqs = [ca.ContextSequence.ordinary(3, 2), ca.ContextSequence.ordinary(0, 4)]
    plan = ca.ContextAttentionPlan.merge(seqs)
    qo, kv, occ, qpos, kpos = (plan.packed[a:b].numpy() for a, b in plan.field_ranges)
    np.testing.assert_array_equal(qo, [0, 2, 6])
    np.testing.assert_array_equal(kv, [0, 3, 3])
    np.testing.assert_array_equal(occ, [0, 1, 2])
    np.testing.assert_array_equal(qpos, [3, 4, 0, 1, 2, 3])
    np.testing.assert_array_equal(kpos, [0, 1, 2])
    assert plan.occurrence_count == 9 and plan.query_lengths == (2, 4)
    assert all(a % 2 == 0 for a, _ in plan.field_ranges)  # 16-byte aligned fields


def test_validation_messages():
    with pytest.raises(ValueError, match="cannot be empty"):
        ca.ContextAttentionPlan.merge([])
    with pytest.raises(ValueError, match="Invalid ordinary"):
        ca.ContextSequence.ordinary(0, 0)
    plan = ca.ContextAttentionPlan.merge([ca.ContextSequence.ordinary(2, 2)])
    with pytest.raises(ValueError, match="must cover all batch occurrences"):
        plan.bind(torch.zeros(3, dtype=torch.int64))
    q = torch.zeros((4, 8, 64), dtype=torch.bfloat16)
    k = torch.zeros((4, 1, 64), dtype=torch.bfloat16)
    ind = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(ValueError, match="both query and KV positions"):
        ca.extend_attention_fwd(q, k, k, q, k, k, ind, ind, ind, None, True, None, 4,
                                context_q_positions=torch.zeros(4, dtype=torch.int64))
    with pytest.raises(ValueError, match="must align with Q/KV"):
        ca.extend_attention_fwd(q, k, k, q, k, k, ind, ind, ind, None, True, None, 4,
                                context_q_positions=torch.zeros(3, dtype=torch.int64),
                                context_kv_positions=torch.zeros(2, dtype=torch.int64))
    with pytest.raises(ValueError, match="requires page_size=1"):
        ca.extend_attention_fwd(q, k, k, q, k, k, ind, ind, ind, None, True, None, 4, page_size=16,
                                context_q_positions=torch.zeros(4, dtype=torch.int64),
                                context_kv_positions=torch.zeros(2, dtype=torch.int64))
    with pytest.raises(ValueError, match="custom mask"):
        ca.extend_attention_fwd(q, k, k, q, k, k, ind, ind, ind, torch.ones(1), True, None, 4)


def test_from_window_checks_segment_shape():
    class W:
        segment_query_starts = np.array([0, 3])
        segment_query_ends = np.array([3, 5])
        occurrence_raw_tokens = np.array([0, 1, 2, 3, 4, 1])
        occurrence_positions = np.array([0, 1, 2, 3, 4, 0])
        birth_occurrences = np.arange(5)
        segment_key_occurrences = np.array([0, 1, 2, 5, 3, 4])
        segment_key_offsets = np.array([0, 3, 6])

    seq = ca.ContextSequence.from_window(W)
    assert seq.query_lengths == (3, 2)
    np.testing.assert_array_equal(seq.prefix_offsets, [0, 0, 1])
    np.testing.assert_array_equal(seq.prefix_occurrences, [5])
    np.testing.assert_array_equal(seq.prefix_positions, [0])
    np.testing.assert_array_equal(seq.query_positions, [0, 1, 2, 3, 4])
    W.segment_query_ends = np.array([3, 3])
    with pytest.raises(ValueError, match="nonempty query segments"):
        ca.ContextSequence.from_window(W)
