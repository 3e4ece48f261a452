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

from dataclasses import dataclass, field, replace

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
# one rank's share of GPT-OSS-120B at tensor parallel 2 (4 of the 8 KV heads)
GPT_OSS_120B_TP2 = Model(
    "gpt-oss-120b TP=2 rank (36 layers, 4 KV heads, head_dim 64, YaRN)",
    36, 4, 64, 64,
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

LLAMA3_8B_2L = replace(LLAMA3_8B, name="llama-3-8b shape with 2 layers", n_layers=2)


@dataclass(frozen=True)
class Workload:
    name: str
    model: Model
    lengths: tuple  # raw tokens per request
    spans: tuple  # per request: tuple of (start, end) dropped ranges
    seed: int
    table_positions: int
    pool_slots: int
    page_size: int = 1
    shared_prefix: int = 0  # raw tokens [0, shared_prefix) of every request share pages

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
    free = kept - max(k - 1, 0)
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


def shared_prefix_workload(name, model, n_requests, prefix, suffix_lo, suffix_hi, k_lo, k_hi, span_lo,
                           span_hi, page_size, seed):
    """Requests sharing a page-aligned prefix, each with a private suffix and
    ``k ~ U{k_lo..k_hi}`` dropped spans of ``U[span_lo, span_hi]`` tokens
    placed inside the prefix."""
    if prefix % page_size:
        raise ValueError("the shared prefix must be page aligned")
    rng = np.random.default_rng(seed)
    lengths, spans = [], []
    for _ in range(n_requests):
        suffix = int(rng.integers(suffix_lo, suffix_hi + 1))
        k = int(rng.integers(k_lo, k_hi + 1))
        spans.append(place_spans(rng, prefix, rng.integers(span_lo, span_hi + 1, size=k)))
        lengths.append(prefix + suffix)
    return Workload(name, model, tuple(lengths), tuple(spans), seed, max(lengths), 0, page_size, prefix)


def paged_demand(w):
    """Per request: (kept, first copied page, fresh pages) of a shared-prefix workload."""
    P = w.page_size
    out = []
    for n, spans in zip(w.lengths, w.spans):
        dropped = sum(e - s for s, e in spans)
        kept = n - dropped
        p0 = spans[0][0] // P if spans else -(-n // P)
        out.append((kept, p0, max(0, -(-kept // P) - p0)))
    return out


@dataclass
class PageAssignment:
    shared_pages: np.ndarray  # int32 [prefix / P]
    birth_rows: list  # per request: int32 token slots in raw order
    fresh_pages: list  # per request: int32 pages for its copied logical pages
    pool_pages: int
    groups: tuple  # requests processed together, in order


def assign_pages(w, groups=None):
    """Physical pages of a shared-prefix workload (page 0 is reserved padding).

    Requests run in ``groups`` (default: all at once).  A group's fresh pages
    come first from pages freed by earlier groups -- their private suffix
    pages, and shared pages whose last reference they dropped -- then from
    spare pages, so peak memory is the old pages plus the largest shortfall
    rather than old plus all fresh pages.  Page ids are a seeded permutation.
    """
    P = w.page_size
    B = w.n_requests
    groups = tuple(tuple(g) for g in (groups or [range(B)]))
    if sorted(b for g in groups for b in g) != list(range(B)):
        raise ValueError("groups must cover every request once")
    shared_n = w.shared_prefix // P
    suffix_n = [-(-(n - w.shared_prefix) // P) for n in w.lengths]
    demand = paged_demand(w)

    def simulate(shared, private, spare):
        free, spare_at, fresh = [], 0, [None] * B
        refs = np.full(shared_n, B, dtype=np.int64)
        for g in groups:
            need = sum(demand[b][2] for b in g)
            take = free[:need]
            free = free[need:]
            extra = need - len(take)
            if spare is not None:
                take = take + list(spare[spare_at : spare_at + extra])
            spare_at += extra
            at = 0
            for b in g:
                fresh[b] = np.asarray(take[at : at + demand[b][2]], dtype=np.int32)
                at += demand[b][2]
            for b in g:
                p0 = demand[b][1]
                free.extend(private[b][max(0, p0 - shared_n):])
                refs[min(p0, shared_n):] -= 1
            for p in np.flatnonzero(refs == 0):
                free.append(shared[p])
                refs[p] = -1
        return fresh, spare_at

    _, spare_n = simulate(np.zeros(shared_n, np.int32), [[0] * s for s in suffix_n], None)
    pool_pages = 1 + shared_n + sum(suffix_n) + spare_n
    rng = np.random.default_rng(w.seed + 1000)
    perm = rng.permutation(np.arange(1, pool_pages, dtype=np.int64)).astype(np.int32)
    shared = perm[:shared_n]
    at = shared_n
    private = []
    for s in suffix_n:
        private.append(list(perm[at : at + s]))
        at += s
    fresh, _ = simulate(shared, private, perm[at:])
    rows = []
    for n, priv in zip(w.lengths, private):
        pages = np.concatenate((shared, np.asarray(priv, dtype=np.int32)))
        i = np.arange(n)
        rows.append((pages[i // P].astype(np.int64) * P + i % P).astype(np.int32))
    return PageAssignment(shared, rows, fresh, pool_pages, groups)


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
    if name == "gpt-oss-32k-median":
        # the same request shape at seed 33: its 18192 moved tokens are the
        # median over seeds 2-59 (seed 2 above moves 12064, the fewest)
        return single_request_workload("gpt-oss-120b-32k-seed33", GPT_OSS_120B, 32768, 12, 500, 2000, 0.40,
                                       seed=33)
    if name == "gpt-oss-32k-tp2":
        # the same request and events, one TP=2 rank's 4 KV heads
        return single_request_workload("gpt-oss-120b-32k-tp2-rank", GPT_OSS_120B_TP2, 32768, 12, 500, 2000, 0.40,
                                       seed=2)
    if name == "llama3-cow-16":
        # Llama-3-8B shape, page 16: 16 requests share an 8192-token prefix
        # (512 pages), each adds a private 16384-122880-token suffix and drops
        # 1-3 spans of 64-512 tokens inside the prefix (copy-on-write)
        return shared_prefix_workload("llama3-8b-cow-16x(8k+[16k,120k])", LLAMA3_8B, 16, 8192, 16384, 122880,
                                      1, 3, 64, 512, 16, seed=4)
    if name == "llama3-cow-small":
        # the same events with 2 layers and 256-1024-token suffixes
        return shared_prefix_workload("llama3-8b-2l-cow-16x(8k+[256,1024])", LLAMA3_8B_2L, 16, 8192, 256,
                                      1024, 1, 3, 64, 512, 16, seed=4)
    if name == "ragged-64":
        # 64 requests of 2048-65536 tokens, 1-8 spans dropping 10-60% each
        return ragged_batch_workload("ragged-64x[2k,64k]", GPT_OSS_120B, 64, 2048, 65536, 1, 8, 0.10,
                                     0.60, seed=3)
    raise ValueError(f"unknown workload {name!r}")


def trajectory_events(n, turns, lo, hi, seed):
    """A multi-turn agent prompt compiled in one prefill: at each of ``turns-1``
    turn boundaries (evenly spaced insertion points) 1-2 tool-output spans of
    ``U[lo, hi]`` tokens inside the previous turn are dropped and the context
    is repositioned.  Returns the event tensors and ``visible_until`` (a
    dropped token is readable by the queries before its drop)."""
    rng = np.random.default_rng(seed)
    bounds = [n * t // turns for t in range(1, turns)]
    inserts, offsets, flat = [], [0], []
    visible = np.full(n, np.iinfo(np.int32).max, dtype=np.int64)
    prev = 0
    for at in bounds:
        k = int(rng.integers(1, 3))
        lengths = rng.integers(lo, hi + 1, size=k)
        if int(lengths.sum()) + k >= at - prev:
            lengths = np.maximum(1, lengths * (at - prev - k - 1) // (int(lengths.sum()) + 1))
        spans = place_spans(rng, at - prev, lengths)
        for s, e in spans:
            flat += [prev + s, prev + e]
            visible[prev + s : prev + e] = at
        inserts.append(at)
        offsets.append(len(flat) // 2)
        prev = at
    events = dict(
        token_ids=torch.arange(n, dtype=torch.int32) % 50000,
        drop_insert_offsets=torch.tensor(inserts, dtype=torch.int32),
        drop_range_offsets=torch.tensor(offsets, dtype=torch.int32),
        drop_ranges=torch.tensor(flat, dtype=torch.int32),
        reposition_raw_boundaries=torch.tensor(inserts, dtype=torch.int32) - 1,
        reposition_insert_offsets=torch.tensor(inserts, dtype=torch.int32),
    )
    return events, torch.from_numpy(visible.astype(np.int32))


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


def assign_slots(w, layouts, order="permutation"):
    """Birth and fresh slots.  ``order="permutation"``: a seeded random
    permutation of the free slots (a fragmented pool, the worst case for the
    Reposition's row accesses); ``"ascending"``: the free list in ascending
    order, what a page-one allocator hands out from an unfragmented pool."""
    if order not in ("permutation", "ascending"):
        raise ValueError(f"unknown slot order {order!r}")
    rng = np.random.default_rng(w.seed + 1000)
    total = sum(w.lengths)
    moved = [int((np.asarray(l.keep_mask) & (np.asarray(l.birth_positions) != np.asarray(l.positions))).sum())
             for l in layouts]
    need = total + sum(moved)
    if need + 1 > w.pool_slots:
        raise ValueError("pool too small for the workload")
    free = np.arange(1, w.pool_slots, dtype=np.int64)
    perm = (rng.permutation(free) if order == "permutation" else free).astype(np.int32)
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
