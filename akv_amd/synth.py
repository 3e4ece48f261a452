"""Seeded synthetic Drop + Reposition workloads (no datasets, no checkpoints).

Each workload is a set of requests whose prompt drops some token spans and
then repositions (both events at insertion ``n``, the shape one agent turn
produces), plus a paged KV pool of random bf16 K/V (N(0, 1), rounded to
nearest even) and a RoPE table.

Span sampler: span lengths are uniform integers in ``[lo, hi]``, redrawn until
their sum is within ``0.01 n`` of ``fraction * n``; the spans are then placed
by a seeded composition of the kept tokens into ``k + 1`` gaps whose interior
gaps are at least one token.  Slot 0 is reserved as padding (a slot ``<= 0``
counts as unmapped); the request's birth slots are a seeded permutation of
the free slots and its fresh slots the next ones in that permutation.
"""

from dataclasses import dataclass, field

import numpy as np
import torch

from .plan import compile_context_layout
from .rope import make_table


@dataclass(frozen=True)
class Model:
    name: str
    n_layers: int
    n_heads: int
    head_dim: int
    rotary_dim: int
    rope: dict
    dtype: torch.dtype = torch.bfloat16
    is_neox_style: bool = True


GPT_OSS_120B = Model(
    "gpt-oss-120b (36 layers, 8 KV heads, head_dim 64, YaRN)",
    36, 8, 64, 64,
    dict(kind="yarn", base=150000.0, factor=32.0, original_max=4096, beta_fast=32.0, beta_slow=1.0),
)
TINY = Model("tiny (2 layers, 2 KV heads, head_dim 64, plain RoPE)", 2, 2, 64, 64,
             dict(kind="plain", base=10000.0))
LLAMA3_8B = Model(
    "llama-3-8b (32 layers, 8 KV heads, head_dim 128, llama3 RoPE)",
    32, 8, 128, 128,
    dict(kind="llama3", base=500000.0, factor=8.0, original_max=8192, low_freq_factor=1.0,
         high_freq_factor=4.0),
)


@dataclass(frozen=True)
class Workload:
    name: str
    model: Model
    lengths: tuple  # raw tokens per request
    spans: tuple  # per request: tuple of (start, end) dropped ranges
    seed: int
    table_positions: int
    pool_slots: int

    @property
    def n_requests(self):
        return len(self.lengths)


def sample_span_lengths(rng, n, k, lo, hi, fraction, tolerance=0.01):
    target = fraction * n
    for _ in range(100000):
        lengths = rng.integers(lo, hi + 1, size=k)
        if abs(int(lengths.sum()) - target) <= tolerance * n:
            return lengths
    raise RuntimeError("span sampler did not converge")


def split_total(rng, total, k):
    """``k`` positive integers summing to ``total`` (uniform composition)."""
    cuts = np.sort(rng.choice(np.arange(1, total), size=k - 1, replace=False)) if k > 1 else []
    edges = np.concatenate(([0], cuts, [total]))
    return np.diff(edges)


def place_spans(rng, n, lengths):
    """Seeded composition of the kept tokens into ``k + 1`` gaps (interior >= 1)."""
    k = len(lengths)
    kept = n - int(np.sum(lengths))
    free = kept - (k - 1)
    if free < 0:
        raise ValueError("spans do not fit")
    # stars and bars: k cut positions among free + k slots
    bars = np.sort(rng.choice(free + k, size=k, replace=False))
    gaps = np.diff(np.concatenate(([-1], bars, [free + k]))) - 1
    gaps[1:k] += 1
    ranges, at = [], 0
    for i, length in enumerate(lengths):
        at += int(gaps[i])
        ranges.append((at, at + int(length)))
        at += int(length)
    assert at + int(gaps[k]) == n
    return tuple(ranges)


def single_request_workload(name, model, n, k, lo, hi, fraction, seed, pool_slots=None):
    rng = np.random.default_rng(seed)
    lengths = sample_span_lengths(rng, n, k, lo, hi, fraction)
    spans = place_spans(rng, n, lengths)
    return Workload(name, model, (n,), (spans,), seed, n, pool_slots or 2 * n + 1)


def ragged_batch_workload(name, model, n_requests, n_lo, n_hi, k_lo, k_hi, f_lo, f_hi, seed):
    rng = np.random.default_rng(seed)
    lengths, spans = [], []
    for _ in range(n_requests):
        n = int(rng.integers(n_lo, n_hi + 1))
        k = int(rng.integers(k_lo, k_hi + 1))
        f = float(rng.uniform(f_lo, f_hi))
        span_lengths = split_total(rng, max(k, int(round(f * n))), k)
        lengths.append(n)
        spans.append(place_spans(rng, n, span_lengths))
    total = sum(lengths)
    return Workload(name, model, tuple(lengths), tuple(spans), seed, max(lengths), 2 * total + 1)


def decode_batch_workload(name, model, n_requests, n, k, lo, hi, fraction, seed0):
    """Requests of equal length, each with its own seeded drop spans (seed0 + b)."""
    spans = []
    for b in range(n_requests):
        rng = np.random.default_rng(seed0 + b)
        spans.append(place_spans(rng, n, sample_span_lengths(rng, n, k, lo, hi, fraction)))
    return Workload(name, model, (n,) * n_requests, tuple(spans), seed0, n, 2 * n * n_requests + 64)


def workload(name):
    """The named synthetic configurations."""
    if name == "gpt-oss-decode-32x32k":
        # 32 GPT-OSS requests of 32768 tokens, 12 spans of 500-2000 dropping
        # ~40% each (seeds 5 + b): the decode consumer check
        return decode_batch_workload("gpt-oss-120b-decode-32x32k", GPT_OSS_120B, 32, 32768, 12, 500, 2000,
                                     0.40, seed0=5)
    if name == "tiny":
        # 2 layers x 2 KV heads x 64, plain RoPE; 4096 tokens, 3 spans of
        # 200-600 tokens dropping 25%
        return single_request_workload("tiny-4k", TINY, 4096, 3, 200, 600, 0.25, seed=1)
    if name == "gpt-oss-32k":
        # GPT-OSS-120B shape; 32768 tokens, 12 tool-result spans of 500-2000
        # tokens dropping ~40%
        return single_request_workload("gpt-oss-120b-32k", GPT_OSS_120B, 32768, 12, 500, 2000, 0.40,
                                       seed=2)
    if name == "ragged-64":
        # 64 requests of 2048-65536 tokens, 1-8 spans dropping 10-60% each
        return ragged_batch_workload("ragged-64x[2k,64k]", GPT_OSS_120B, 64, 2048, 65536, 1, 8, 0.10,
                                     0.60, seed=3)
    raise ValueError(f"unknown workload {name!r}")


def request_events(n, spans):
    """Event tensors of one Drop (all spans) + one Reposition, both at insertion n."""
    flat = [x for span in spans for x in span]
    return dict(
        token_ids=torch.arange(n, dtype=torch.int32) % 50000,
        drop_insert_offsets=torch.tensor([n] if spans else [], dtype=torch.int32),
        drop_range_offsets=torch.tensor([0, len(spans)] if spans else [0], dtype=torch.int32),
        drop_ranges=torch.tensor(flat, dtype=torch.int32),
        reposition_raw_boundaries=torch.tensor([n - 1], dtype=torch.int32),
        reposition_insert_offsets=torch.tensor([n], dtype=torch.int32),
    )


def compile_layouts(w):
    return [compile_context_layout(**request_events(n, s)) for n, s in zip(w.lengths, w.spans)]


@dataclass
class SlotAssignment:
    birth_rows: list  # per request: int32 numpy birth slots in raw order
    fresh: list  # per request: int32 numpy fresh slots (moved tokens, raw order)
    moved: list  # per request: number of moved tokens


def assign_slots(w, layouts):
    rng = np.random.default_rng(w.seed + 1000)
    total = sum(w.lengths)
    moved = [int((np.asarray(l.keep_mask) & (np.asarray(l.birth_positions) != np.asarray(l.positions))).sum())
             for l in layouts]
    need = total + sum(moved)
    if need + 1 > w.pool_slots:
        raise ValueError("pool too small for the workload")
    perm = rng.permutation(np.arange(1, w.pool_slots, dtype=np.int64)).astype(np.int32)
    births, fresh, at = [], [], 0
    for n in w.lengths:
        births.append(perm[at : at + n])
        at += n
    for m in moved:
        fresh.append(perm[at : at + m])
        at += m
    return SlotAssignment(births, fresh, moved)


def rope_table(w, device="cpu", dtype=torch.float32):
    spec = dict(w.model.rope)
    kind = spec.pop("kind")
    return make_table(kind, w.model.rotary_dim, w.table_positions, dtype=dtype, device=device, **spec)


@dataclass
class KVPool:
    k: list = field(default_factory=list)
    v: list = field(default_factory=list)
    k_ptrs: torch.Tensor = None
    v_ptrs: torch.Tensor = None


def make_pool(model, slots, device, seed, *, generate_on_device=None):
    """Per-layer ``[slots, heads, head_dim]`` K/V buffers of N(0, 1) values.

    Small pools are drawn on the CPU (reproducible for the oracle); large
    ones directly on the device.
    """
    shape = (slots, model.n_heads, model.head_dim)
    elements = slots * model.n_heads * model.head_dim * model.n_layers * 2
    on_device = generate_on_device if generate_on_device is not None else elements > (1 << 26)
    pool = KVPool()
    if on_device:
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        for _ in range(model.n_layers):
            pool.k.append(torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(model.dtype))
            pool.v.append(torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(model.dtype))
    else:
        gen = torch.Generator()
        gen.manual_seed(seed)
        for _ in range(model.n_layers):
            pool.k.append(torch.randn(shape, generator=gen, dtype=torch.float32).to(model.dtype).to(device))
            pool.v.append(torch.randn(shape, generator=gen, dtype=torch.float32).to(model.dtype).to(device))
    pool.k_ptrs = torch.tensor([t.data_ptr() for t in pool.k], dtype=torch.uint64).to(device)
    pool.v_ptrs = torch.tensor([t.data_ptr() for t in pool.v], dtype=torch.uint64).to(device)
    return pool
