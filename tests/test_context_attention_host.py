"""Host side of the prefill context attention: the extend entry's
validation messages (no kernel launch), and the tests' metadata helper."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from akv_amd import context_attention as ca

from harness import attention_metadata, plain_segments, window_segments


def test_validation_messages():
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


def test_metadata_helper_splits_segments():
    """Two query segments; the second reads one key (occurrence 5) before
    its own births; a plain request follows with occurrence ids offset."""
    window = SimpleNamespace(
        segment_query_starts=np.array([0, 3]), segment_query_ends=np.array([3, 5]),
        occurrence_raw_tokens=np.array([0, 1, 2, 3, 4, 1]), occurrence_positions=np.array([0, 1, 2, 3, 4, 0]),
        birth_occurrences=np.arange(5), segment_key_occurrences=np.array([0, 1, 2, 5, 3, 4]),
        segment_key_offsets=np.array([0, 3, 6]))
    seg = window_segments(window)
    np.testing.assert_array_equal(seg.query_lengths, [3, 2])
    np.testing.assert_array_equal(seg.prefix_lengths, [0, 1])
    np.testing.assert_array_equal(seg.prefix, [5])
    np.testing.assert_array_equal(seg.prefix_positions, [0])
    np.testing.assert_array_equal(seg.query_positions, [0, 1, 2, 3, 4])
    meta = attention_metadata([seg, plain_segments(3, 2)], torch.arange(100, 111))
    c = meta.cpu
    np.testing.assert_array_equal(c.qo_indptr, [0, 3, 5, 7])
    np.testing.assert_array_equal(c.kv_indptr, [0, 0, 1, 4])
    np.testing.assert_array_equal(c.occurrences, [5, 6, 7, 8])
    np.testing.assert_array_equal(meta.kv_indices.numpy(), [105, 106, 107, 108])
    np.testing.assert_array_equal(c.query_positions, [0, 1, 2, 3, 4, 3, 4])
    np.testing.assert_array_equal(c.kv_positions, [0, 0, 1, 2])
