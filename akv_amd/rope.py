"""RoPE cos/sin tables in the layout the Reposition kernel reads.

``[positions, rotary_dim]``: cos of every rotary frequency in the first half,
sin in the second (the layout of the model's ``cos_sin_cache``, read at
``akv/system/sglang/kernels/ops/attention/context_reposition.py:82-91``).
Frequencies and angles are computed in fp32 as a model's rotary module does:
``inv_freq[i] = base ** (-2i / R)``, ``angle = position * inv_freq``.

Scalings:

* ``plain``  -- unscaled rotary embedding (RoFormer).
* ``yarn``   -- YaRN (Peng et al., 2023, arXiv:2309.00071): per-frequency
  blend of interpolated (``inv_freq / factor``) and extrapolated
  (``inv_freq``) frequencies with a linear ramp between the correction dims
  of ``beta_fast`` and ``beta_slow`` rotations over the original context;
  cos and sin multiplied by ``mscale = 0.1 ln(factor) + 1``.
* ``llama3`` -- Llama 3.1 frequency scaling: wavelengths above
  ``orig_ctx / low_freq_factor`` divided by ``factor``, below
  ``orig_ctx / high_freq_factor`` unchanged, smooth interpolation between.

The table provider of the reference lives in the serving engine, not in the
reference repository; these generators are checked against the published
formulas (and the ``transformers`` implementations of them) in the tests.
Parity against the engine's own rotary modules is unpinned (absent here);
the Reposition kernel and the oracle read the same table, so the kernel's
parity holds for any table.
"""

import math

import torch


def plain_inv_freq(rotary_dim, base):
    return 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))


def _correction_dim(rotations, rotary_dim, base, original_max):
    return (rotary_dim * math.log(original_max / (rotations * 2 * math.pi))) / (2 * math.log(base))


def yarn_inv_freq(rotary_dim, base, factor, original_max, beta_fast=32.0, beta_slow=1.0,
                  truncate=True):
    pos_freqs = base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim)
    extrapolated = 1.0 / pos_freqs
    interpolated = 1.0 / (factor * pos_freqs)
    low = _correction_dim(beta_fast, rotary_dim, base, original_max)
    high = _correction_dim(beta_slow, rotary_dim, base, original_max)
    if truncate:
        low, high = math.floor(low), math.ceil(high)
    low, high = max(low, 0), min(high, rotary_dim - 1)
    if low == high:
        high += 0.001
    ramp = torch.clamp((torch.arange(rotary_dim // 2, dtype=torch.float32) - low) / (high - low), 0, 1)
    keep_extrapolated = 1 - ramp
    return interpolated * (1 - keep_extrapolated) + extrapolated * keep_extrapolated


def yarn_mscale(factor):
    return 1.0 if factor <= 1 else 0.1 * math.log(factor) + 1.0


def llama3_inv_freq(rotary_dim, base, factor, original_max, low_freq_factor=1.0,
                    high_freq_factor=4.0):
    inv_freq = plain_inv_freq(rotary_dim, base)
    low_wavelen = original_max / low_freq_factor
    high_wavelen = original_max / high_freq_factor
    wavelen = 2 * math.pi / inv_freq
    scaled = torch.where(wavelen > low_wavelen, inv_freq / factor, inv_freq)
    smooth = (original_max / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    smoothed = (1 - smooth) * scaled / factor + smooth * scaled
    medium = (wavelen >= high_wavelen) & (wavelen <= low_wavelen)
    return torch.where(medium, smoothed, scaled)


def cos_sin_table(inv_freq, positions, scale=1.0, dtype=torch.float32, device="cpu"):
    """``[positions, 2 * len(inv_freq)]`` table: cos | sin, times ``scale``."""
    t = torch.arange(positions, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq.to(torch.float32))
    cos = freqs.cos()
    sin = freqs.sin()
    if scale != 1.0:
        cos = cos * scale
        sin = sin * scale
    return torch.cat((cos, sin), dim=-1).to(dtype=dtype, device=device).contiguous()


def make_table(kind, rotary_dim, positions, *, base, factor=1.0, original_max=None,
               dtype=torch.float32, device="cpu", **kw):
    """Build a plain / YaRN / llama3 table of ``positions`` rows."""
    if kind == "plain":
        return cos_sin_table(plain_inv_freq(rotary_dim, base), positions, dtype=dtype, device=device)
    if kind == "yarn":
        inv = yarn_inv_freq(rotary_dim, base, factor, original_max, **kw)
        return cos_sin_table(inv, positions, scale=yarn_mscale(factor), dtype=dtype, device=device)
    if kind == "llama3":
        inv = llama3_inv_freq(rotary_dim, base, factor, original_max, **kw)
        return cos_sin_table(inv, positions, dtype=dtype, device=device)
    raise ValueError(f"unknown RoPE scaling {kind!r}")
