"""RoPE table generators against the published formulas as implemented in
transformers (a library routine the reference's model code also follows)."""

import math
from types import SimpleNamespace

import pytest
import torch

from akv_amd import rope

transformers_rope = pytest.importorskip("transformers.modeling_rope_utils")


def _config(rope_type, theta, head_dim, **params):
    parameters = dict(rope_type=rope_type, rope_theta=theta, **params)
    cfg = SimpleNamespace(
        rope_parameters=parameters,
        rope_scaling=parameters,
        rope_theta=theta,
        head_dim=head_dim,
        hidden_size=head_dim * 8,
        num_attention_heads=8,
        max_position_embeddings=params.get("original_max_position_embeddings", 4096) * 32,
        partial_rotary_factor=1.0,
        default_theta=theta,
    )
    cfg.standardize_rope_params = lambda *a, **k: None
    return cfg


def _hf(rope_type, cfg):
    fn = transformers_rope.ROPE_INIT_FUNCTIONS[rope_type]
    return fn(cfg, "cpu")


@pytest.mark.parametrize("truncate", [True, False])
def test_yarn_matches_transformers(truncate):
    cfg = _config("yarn", 150000.0, 64, factor=32.0, original_max_position_embeddings=4096,
                  beta_fast=32.0, beta_slow=1.0, truncate=truncate)
    try:
        inv, scale = _hf("yarn", cfg)
    except Exception as err:  # config protocol differs across versions
        pytest.skip(f"transformers yarn init unavailable: {err}")
    mine = rope.yarn_inv_freq(64, 150000.0, 32.0, 4096, 32.0, 1.0, truncate=truncate)
    torch.testing.assert_close(mine, inv.float(), rtol=0, atol=0)
    assert scale == pytest.approx(rope.yarn_mscale(32.0), rel=1e-12)
    assert rope.yarn_mscale(32.0) == pytest.approx(0.1 * math.log(32) + 1)


def test_llama3_matches_transformers():
    cfg = _config("llama3", 500000.0, 128, factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                  original_max_position_embeddings=8192)
    try:
        inv, scale = _hf("llama3", cfg)
    except Exception as err:
        pytest.skip(f"transformers llama3 init unavailable: {err}")
    mine = rope.llama3_inv_freq(128, 500000.0, 8.0, 8192, 1.0, 4.0)
    torch.testing.assert_close(mine, inv.float(), rtol=1e-7, atol=0)
    assert scale == 1.0


def test_plain_closed_form_and_layout():
    t = rope.make_table("plain", 8, 5, base=10000.0)
    assert t.shape == (5, 8)
    inv = [10000.0 ** (-2 * i / 8) for i in range(4)]
    for p in range(5):
        for i in range(4):
            assert float(t[p, i]) == pytest.approx(math.cos(p * inv[i]), abs=1e-6)
            assert float(t[p, 4 + i]) == pytest.approx(math.sin(p * inv[i]), abs=1e-6)
    y = rope.make_table("yarn", 64, 4, base=150000.0, factor=32.0, original_max=4096)
    # |(cos, sin)| = mscale for YaRN
    norm = (y[:, :32] ** 2 + y[:, 32:] ** 2).sqrt()
    torch.testing.assert_close(norm, torch.full_like(norm, rope.yarn_mscale(32.0)), rtol=1e-5, atol=0)
