"""Benchmark: Drop + Reposition of retained KV on one MI355X.

Workload: one GPT-OSS-120B-shaped request (36 layers, 8 KV heads, head_dim
64, bf16 K/V ~ N(0, 1), YaRN RoPE theta 150000 / factor 32 / original 4096,
page size 1) of 32768 tokens dropping 12 seeded spans (~40%), then one
Reposition.  Synthetic data; all inputs resident in HBM before timing.

One step = the whole GPU side of the hot path as a caller runs it:
page-table compaction (terminal row, freed slots, copy lists, decode layout,
kv_indptr / kv_indices; 2 launches) -> all-layer Reposition (K re-rotation +
V move, one launch) gated on the device by the compaction's status word.  No
host read or sync sits between them, in the product or here.  ``value`` =
retained-KV bytes moved (K and V, read + write) per step / step time over K
back-to-back steps.  Also reported: the Reposition
kernel's average launch in that timed region and its roofline against
8 TB/s; p50 / p99 latency of the step and of the Reposition alone after a
1 GiB read flush of L2 + the 256 MB MALL; the CPU oracle on a bounded sample
of the same workload.  ``other_configs`` measures the surrounding rows on
their own workloads: the tiny and ragged-batch compactions, ascending slots,
one TP=2 rank's head share,
the decode step over the compacted metadata, the next turn's prefill
attention (GPT-OSS and Llama-3 layer shapes), a multi-turn trajectory's
occurrence binding in one forward and in 4 chunked forwards, the
compacted handoff copies and the page-16 copy-on-write batch.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from akv_amd import _lib, ops, synth, tables  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "Reposition retained-KV GB/s (% HBM peak) + p50 latency, 32k GPT-OSS-shaped"
PMC_SUMMARY = ROOT / "profiles" / "reposition_gpt-oss-32k_pmc.txt"


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="gpt-oss-32k")
    p.add_argument("--latency-iters", type=int, default=100)
    p.add_argument("--cpu-runs", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-cow", action="store_true", help="skip the page-16 copy-on-write configuration")
    p.add_argument("--reposition-only", action="store_true",
                   help="time only the Reposition launch (for profiling runs)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only copy 1 GiB -> 1 GiB three times (scales rocprof byte counters)")
    p.add_argument("--only", choices=["handoff", "prefill", "prefill-llama", "chunked", "decode", "ragged"],
                   help="run one secondary configuration alone and print its line (for profiling runs)")
    return p.parse_args()


def copy_calibration(device):
    src = torch.ones(1 << 28, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4}))


class Pipeline:
    def __init__(self, name, device, slot_order="permutation"):
        self.device = device
        self.w_name = name
        w = self.w = synth.workload(name)
        if w.n_requests != 1:
            raise SystemExit("the bench workload must be a single request")
        m = w.model
        t0 = time.perf_counter()
        self.layouts = synth.compile_layouts(w)
        self.compile_s = time.perf_counter() - t0
        lay = self.layouts[0]
        slots = synth.assign_slots(w, self.layouts, slot_order)
        self.slots = slots
        n = w.lengths[0]
        self.n = n
        self.moved = slots.moved[0]
        self.kept = int(lay.keep_mask.sum())
        # request table row 1 receives the terminal row; the birth slots (the
        # prefill's allocated slots) come as their own vector, so every step
        # reads identical inputs
        table = torch.full((2, n + 8), -1, dtype=torch.int32)
        table[1, n] = int(slots.fresh[0][0])  # first generated token's slot
        self.table = table.to(device)
        self.birth = torch.from_numpy(slots.birth_rows[0]).to(device)
        self.rows = torch.tensor([1], dtype=torch.int64, device=device)
        self.inputs = tables.pack_compaction_inputs(self.layouts, device)
        self.out = tables.allocate_outputs(self.inputs, device, generated_total=1)
        self.generated = torch.ones(1, dtype=torch.int32, device=device)
        self.fresh = torch.from_numpy(slots.fresh[0]).to(device)
        self.pool = synth.make_pool(m, w.pool_slots, device, seed=0, generate_on_device=True)
        self.rope = synth.rope_table(w, device)
        self.stream = torch.cuda.current_stream(device)
        # scratch that evicts the 256 MB MALL between timed iterations
        self.flush_buf = torch.ones(1 << 28, dtype=torch.float32, device=device)
        self.flush_out = torch.empty((), dtype=torch.float32, device=device)
        kv_bytes = 2  # bf16
        self.retained_bytes = self.moved * 4 * m.n_layers * m.n_heads * m.head_dim * kv_bytes
        self.alg_bytes = self.retained_bytes + self.moved * 16 + self.moved * 2 * m.rotary_dim * 4
        # the lists exist from construction on (a gated Reposition of outputs
        # no compaction wrote would do nothing; an ungated one would read
        # uninitialised slots)
        self.compaction()

    def compaction(self):
        tables.compact_rows(self.inputs, self.table, self.rows, self.fresh, self.out, generated=self.generated,
                            birth_slots=self.birth)

    def reposition(self):
        # gated on the device by the compaction's status word: the lists go
        # from the compaction to the Reposition with no host read
        p, o = self.pool, self.out
        ops.reposition_kv_layers_gated(p.k_ptrs, p.v_ptrs, p.k[0], p.v[0], o.copy_src, o.copy_dst, o.copy_pairs,
                                       self.rope, status=o.status, is_neox_style=self.w.model.is_neox_style)

    def step(self):
        self.compaction()
        self.reposition()

    def flush(self):
        # read 1 GiB: evicts the MALL and L2 with clean lines, so the timed
        # kernel neither hits warm data nor pays for unrelated write-backs
        torch.sum(self.flush_buf, 0, out=self.flush_out)


def _time_steps(fn, steps, warmup, iters, flush):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    warm = a.elapsed_time(b) / steps
    cold = []
    for _ in range(iters):
        flush()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        cold.append(a.elapsed_time(b))
    return warm, cold


def _graph_steps(fn, steps):
    """Back-to-back replays of the step captured once in a HIP graph (no host
    launch overhead between kernels); the step allocates nothing and records
    no memset."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def tiny_config(device, flush):
    """2 layers x 2 KV heads x 64, 4096 tokens: cache-resident, latency-bound."""
    pipe = Pipeline("tiny", device)
    warm, cold = _time_steps(pipe.step, 50, 10, 50, flush)
    graph = _graph_steps(pipe.step, 50)
    return {
        "workload": pipe.w.name, "tokens": pipe.n, "moved": pipe.moved,
        "step_ms_back_to_back": round(warm, 5), "step_ms_graph_replay": round(graph, 5),
        "step_p50_ms": round(percentile(cold, 50), 5),
        "step_p99_ms": round(percentile(cold, 99), 5),
        "kernel_launches_per_step": compaction_launches(pipe.inputs) + 1,
    }


def ascending_slots_config(device, flush):
    """The 32k GPT-OSS step with slots from an unfragmented ascending free
    list instead of a random permutation: same tokens, spans and bytes."""
    pipe = Pipeline("gpt-oss-32k", device, slot_order="ascending")
    warm, cold = _time_steps(pipe.step, 50, 10, 50, flush)
    repo_warm, _ = _time_steps(pipe.reposition, 50, 10, 0, flush)
    out = {
        "workload": pipe.w.name + ", ascending slots", "moved": pipe.moved,
        "step_ms_back_to_back": round(warm, 5), "step_p50_ms": round(percentile(cold, 50), 5),
        "retained_kv_GBs": round(pipe.retained_bytes / (warm / 1e3) / 1e9, 1),
        "reposition_ms": round(repo_warm, 5),
        "reposition_pct_hbm_peak": round(100 * pipe.alg_bytes / (repo_warm / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
    }
    del pipe
    return out


def median_moved_config(device, flush):
    """The 32k GPT-OSS request at the median moved count over drop-span
    seeds (seed 33, 18192 moved tokens; the headline seed moves 12064, the
    fewest of seeds 2-59): same shape, span sampler and byte accounting."""
    pipe = Pipeline("gpt-oss-32k-median", device)
    warm, cold = _time_steps(pipe.step, 50, 10, 50, flush)
    repo_warm, _ = _time_steps(pipe.reposition, 50, 10, 0, flush)
    out = {
        "workload": pipe.w.name, "moved": pipe.moved,
        "step_ms_back_to_back": round(warm, 5), "step_p50_ms": round(percentile(cold, 50), 5),
        "retained_kv_GBs": round(pipe.retained_bytes / (warm / 1e3) / 1e9, 1),
        "reposition_ms": round(repo_warm, 5),
        "reposition_pct_hbm_peak": round(100 * pipe.alg_bytes / (repo_warm / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
    }
    del pipe
    torch.cuda.empty_cache()
    return out


def tp2_share_config(device, flush):
    """One rank's share of the 32k GPT-OSS step at tensor parallel 2: the
    same tokens and spans, 4 of the 8 KV heads (512 B K and V rows)."""
    pipe = Pipeline("gpt-oss-32k-tp2", device)
    warm, cold = _time_steps(pipe.step, 50, 10, 50, flush)
    repo_warm, _ = _time_steps(pipe.reposition, 50, 10, 0, flush)
    out = {
        "workload": pipe.w.name, "moved": pipe.moved,
        "step_ms_back_to_back": round(warm, 5), "step_p50_ms": round(percentile(cold, 50), 5),
        "retained_kv_GBs": round(pipe.retained_bytes / (warm / 1e3) / 1e9, 1),
        "reposition_ms": round(repo_warm, 5),
        "reposition_pct_hbm_peak": round(100 * pipe.alg_bytes / (repo_warm / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
    }
    del pipe
    torch.cuda.empty_cache()
    return out


def ragged_config(device, flush):
    """64 requests of 2k-64k tokens: batched compaction + kv_indptr / kv_indices / last-page rebuild."""
    w = synth.workload("ragged-64")
    t0 = time.perf_counter()
    layouts = synth.compile_layouts(w)
    compile_ms = (time.perf_counter() - t0) * 1e3
    slots = synth.assign_slots(w, layouts)
    inputs = tables.pack_compaction_inputs(layouts, device)
    table = torch.full((w.n_requests, max(w.lengths) + 8), -1, dtype=torch.int32, device=device)
    birth = torch.from_numpy(np.concatenate(slots.birth_rows)).to(device)
    fresh = torch.from_numpy(np.concatenate(slots.fresh)).to(device)
    out = tables.allocate_outputs(inputs, device, generated_total=w.n_requests)
    gen = torch.ones(w.n_requests, dtype=torch.int32, device=device)
    rows = torch.arange(w.n_requests, dtype=torch.int64, device=device)

    def step():
        tables.compact_rows(inputs, table, rows, fresh, out, generated=gen, birth_slots=birth)

    warm, cold = _time_steps(step, 50, 10, 50, flush)
    graph = _graph_steps(step, 50)
    status = tables.check_status(out)  # after timing: the outputs were complete
    total = sum(w.lengths)
    # bytes: keep + positions + birth slot read, row write, lists written
    meta = total * (1 + 8 + 4 + 4) + 4 * inputs.retired_total + 16 * inputs.moved_total \
        + 8 * inputs.kept_total + 4 * (inputs.kept_total + w.n_requests) + 12 * w.n_requests
    return {
        "workload": w.name, "requests": w.n_requests, "tokens": total, "kept": inputs.kept_total,
        "moved": inputs.moved_total, "step_ms_back_to_back": round(warm, 5),
        "step_ms_graph_replay": round(graph, 5),
        "step_p50_ms": round(percentile(cold, 50), 5), "step_p99_ms": round(percentile(cold, 99), 5),
        "kernel_launches_per_step": compaction_launches(inputs), "compaction_passes": compaction_passes(inputs),
        "status": status, "metadata_bytes": meta, "host_event_compile_ms": round(compile_ms, 1),
    }


def decode_consumer_config(device, flush):
    """GPT-OSS decode step (32 requests x 32k, 64 q / 8 KV heads, sinks) over the
    compacted metadata: full layer and 128-token sliding-window layer."""
    import dataclasses

    from akv_amd import attention, page_table

    w = synth.workload("gpt-oss-decode-32x32k")
    model = dataclasses.replace(w.model, n_layers=2)
    layouts = synth.compile_layouts(w)
    slots = synth.assign_slots(w, layouts)
    B, n = w.n_requests, w.lengths[0]
    used = np.concatenate(slots.birth_rows + slots.fresh)
    gen_slot = np.setdiff1d(np.arange(1, w.pool_slots), used)[:B].astype(np.int32)
    table = torch.full((B, n + 4), -1, dtype=torch.int32)
    table[:, n] = torch.from_numpy(gen_slot)
    table = table.to(device)
    inputs = tables.pack_compaction_inputs(layouts, device)
    out = tables.allocate_outputs(inputs, device, generated_total=B)
    rows = torch.arange(B, dtype=torch.int64, device=device)
    tables.compact_rows(inputs, table, rows, torch.from_numpy(np.concatenate(slots.fresh)).to(device), out,
                        generated=torch.ones(B, dtype=torch.int32, device=device),
                        birth_slots=torch.from_numpy(np.concatenate(slots.birth_rows)).to(device))
    pool = synth.make_pool(model, w.pool_slots, device, seed=9, generate_on_device=True)

    # registry rows (the reference registry's row format) straight from the
    # compaction outputs: raw indices and positions of the active versions
    kept_off = np.concatenate(([0], np.cumsum(inputs.kept)))
    registry = torch.tensor(
        [(out.raw_indices.data_ptr() + 4 * int(kept_off[b]), out.active_positions.data_ptr() + 4 * int(kept_off[b]),
          n, inputs.kept[b], layouts[b].next_position, 0) for b in range(B)], dtype=torch.int64).to(device)
    seq = torch.tensor([k + 1 for k in inputs.kept], dtype=torch.int64, device=device)
    win_indptr = torch.zeros(B + 1, dtype=torch.int32, device=device)
    win_idx = torch.zeros(B * 129, dtype=torch.int32, device=device)
    win_len = torch.empty_like(seq)
    win_start = torch.empty_like(seq)

    def meta_window():
        page_table.context_window_lengths(registry, rows, seq, win_len, 128, starts=win_start)
        page_table.build_indptr(win_len, win_indptr)
        page_table.context_decode_indices(registry, table, rows, win_len, win_indptr, win_idx, starts=win_start,
                                          status=out.status)

    meta_window()
    q = torch.randn((B, 64, 64), device=device).to(torch.bfloat16)
    sinks = torch.randn(64, device=device)
    o = torch.empty((B, 64, 64), dtype=torch.bfloat16, device=device)
    max_full = max(inputs.kept) + 1
    ws = torch.empty(attention.workspace_bytes(B, 8, 64, max_full) // 4 + 1, dtype=torch.float32, device=device)

    def full():
        attention.decode_attention(q, pool.k[1], pool.v[1], out.kv_indptr, out.kv_indices, o, scale=0.125,
                                   max_len=max_full, sinks=sinks, workspace=ws, status=out.status)

    def windowed():
        attention.decode_attention(q, pool.k[0], pool.v[0], win_indptr, win_idx, o, scale=0.125, max_len=129,
                                   sinks=sinks, workspace=ws, status=out.status)

    # the step's own read metadata from the registry: kv_indptr + kv_indices
    # for the full layer, window lengths + indptr + indices for the SWA layer
    meta_indptr = torch.zeros(B + 1, dtype=torch.int32, device=device)
    meta_idx = torch.full((inputs.kept_total + B,), -1, dtype=torch.int32, device=device)

    def meta_full():
        page_table.build_indptr(seq, meta_indptr)
        page_table.context_decode_indices(registry, table, rows, seq, meta_indptr, meta_idx, status=out.status)

    meta_full()
    tables.check_status(out)  # a check of this run, after the gated consumers
    if not (torch.equal(meta_indptr, out.kv_indptr.to(torch.int32)) and torch.equal(meta_idx, out.kv_indices)):
        raise RuntimeError("decode read indices disagree with the compaction's kv_indices")
    warm_meta_full, cold_meta_full = _time_steps(meta_full, 50, 5, 20, flush)
    warm_meta_win, cold_meta_win = _time_steps(meta_window, 50, 5, 20, flush)
    warm_full, cold_full = _time_steps(full, 20, 5, 20, flush)
    warm_win, cold_win = _time_steps(windowed, 50, 5, 20, flush)
    keys = inputs.kept_total + B
    kv_bytes = keys * 8 * 64 * 2 * 2  # K and V rows of 8 KV heads
    return {
        "workload": w.name + " decode step (64 q / 8 KV heads, sinks)",
        "keys_full_layer": keys,
        "full_layer_ms": round(warm_full, 5), "full_layer_p50_ms": round(percentile(cold_full, 50), 5),
        "full_layer_kv_GBs": round(kv_bytes / (warm_full / 1e3) / 1e9, 1),
        "window128_layer_ms": round(warm_win, 5), "window128_layer_p50_ms": round(percentile(cold_win, 50), 5),
        # split over key chunks + combine; a window layer's keys fit one chunk
        "kernel_launches_per_layer": {"full": 2, "window128": 1},
        "metadata": {
            "full_ms": round(warm_meta_full, 5), "full_p50_ms": round(percentile(cold_meta_full, 50), 5),
            "full_p99_ms": round(percentile(cold_meta_full, 99), 5),
            "window128_ms": round(warm_meta_win, 5),
            "window128_p50_ms": round(percentile(cold_meta_win, 50), 5),
            "window128_p99_ms": round(percentile(cold_meta_win, 99), 5),
            "kernel_launches": {"full": 2, "window128": 3},
        },
    }


def cow_config(device, flush):
    """Llama-3-8B page-16 copy-on-write: 16 requests over a shared 8192-token
    prefix with 16k-120k private suffixes.  Requests run in the fewest groups
    whose pool (old pages + the fresh pages not covered by pages the earlier
    groups released) fits the free HBM; per group one paged compaction and
    one all-layer Reposition."""
    w = synth.workload("llama3-cow-16")
    m = w.model
    P = w.page_size
    t0 = time.perf_counter()
    layouts = synth.compile_layouts(w)
    compile_ms = (time.perf_counter() - t0) * 1e3
    torch.cuda.empty_cache()
    free, _ = torch.cuda.mem_get_info(device)
    page_bytes = P * m.n_layers * m.n_heads * m.head_dim * 2 * 2
    assignment = None
    for n_groups in (1, 2, 4, 8, 16):
        size = w.n_requests // n_groups
        a = synth.assign_pages(w, [range(i, i + size) for i in range(0, w.n_requests, size)])
        if a.pool_pages * page_bytes < free - (12 << 30):
            assignment = a
            break
    if assignment is None:
        return {"workload": w.name, "skipped": f"pool does not fit {free / 2**30:.0f} GiB of free HBM"}
    a = assignment
    pool = synth.make_pool(m, a.pool_pages * P, device, seed=4, generate_on_device=True)
    rope = synth.rope_table(w, device)
    table = torch.full((w.n_requests, max(w.lengths) + 8), -1, dtype=torch.int32, device=device)
    groups = []
    for g in a.groups:
        g = list(g)
        inp = tables.pack_paged_inputs([layouts[b] for b in g], P, device)
        groups.append(dict(
            inputs=inp, out=tables.allocate_paged_outputs(inp, device),
            rows=torch.tensor(g, dtype=torch.int64, device=device),
            fresh=torch.from_numpy(np.concatenate([a.fresh_pages[b] for b in g])).to(device),
            birth=torch.from_numpy(np.concatenate([a.birth_rows[b] for b in g])).to(device),
            events=[],
        ))
    copies = sum(sum(gr["inputs"].copies) for gr in groups)

    def step(record=False):
        for gr in groups:
            tables.compact_pages(gr["inputs"], table, gr["rows"], gr["fresh"], gr["out"], birth_slots=gr["birth"])
            o = gr["out"]
            if record:
                e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                e[0].record()
            ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], o.copy_src, o.copy_dst,
                                     o.copy_pairs, rope)
            if record:
                e[1].record()
                gr["events"].append(e)

    warm, cold = _time_steps(step, 10, 2, 5, flush)
    for gr in groups:
        gr["events"].clear()
    step(record=True)
    step(record=True)
    torch.cuda.synchronize()
    repo_ms = sum(float(np.mean([b.elapsed_time(e) for b, e in gr["events"]])) for gr in groups)
    retained = copies * 4 * m.n_layers * m.n_heads * m.head_dim * 2
    alg = retained + copies * 16 + copies * 2 * m.rotary_dim * 4
    del pool
    torch.cuda.empty_cache()
    return {
        "workload": w.name, "requests": w.n_requests, "tokens": sum(w.lengths), "copies": copies,
        "page_size": P, "groups": len(a.groups), "pool_GiB": round(a.pool_pages * page_bytes / 2**30, 1),
        "step_ms_back_to_back": round(warm, 4), "step_p50_ms": round(percentile(cold, 50), 4),
        "retained_kv_GBs": round(retained / (warm / 1e3) / 1e9, 1),
        "reposition_ms_per_step": round(repo_ms, 4),
        "reposition_pct_hbm_peak": round(100 * alg / (repo_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
        "kernel_launches_per_step": 2 * len(a.groups), "host_event_compile_ms": round(compile_ms, 1),
    }


def multistage_config(device, flush):
    """A 6-turn agent prompt of 32768 tokens compiled in one prefill (1-2
    dropped tool spans of 500-2000 tokens per turn boundary): host layout and
    occurrence-window compile (C++), then the device binding of every
    occurrence (slots, copies, terminal row, retired slots; 2 launches) and
    the all-layer Reposition of the copies."""
    from akv_amd import occurrence as ow
    from akv_amd import plan

    n = 32768
    events, visible = synth.trajectory_events(n, 6, 500, 2000, seed=6)
    t0 = time.perf_counter()
    lay = plan.compile_context_layout(**events)
    t1 = time.perf_counter()
    window = ow.compile_occurrence_window(lay, visible, lay.positions, query_start=0, query_end=n)
    t2 = time.perf_counter()
    keep = np.asarray(lay.keep_mask, dtype=bool)
    inp = ow.pack_final_forward([window], [keep], device)
    t3 = time.perf_counter()
    out = ow.allocate_final_forward_outputs(inp, device)
    m = synth.GPT_OSS_120B
    pool_slots = n + inp.extra[0] + 1
    rng = np.random.default_rng(6)
    perm = rng.permutation(np.arange(1, pool_slots)).astype(np.int32)
    birth = torch.from_numpy(perm[:n]).to(device)
    fresh = torch.from_numpy(perm[n:]).to(device)
    table = torch.full((1, n + 8), -1, dtype=torch.int32, device=device)
    rows = torch.zeros(1, dtype=torch.int64, device=device)
    pool = synth.make_pool(m, pool_slots, device, seed=6, generate_on_device=True)
    w = synth.Workload("trajectory", m, (n,), ((),), 6, 2 * n, pool_slots)
    rope = synth.rope_table(w, device)

    def bind():
        ow.bind_final_forward(inp, table, rows, birth, fresh, out)

    def repo():
        ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], out.copy_src, out.copy_dst,
                                 out.copy_pairs, rope)

    bind()
    warm_bind, cold_bind = _time_steps(bind, 50, 5, 20, flush)
    warm_repo, _ = _time_steps(repo, 20, 3, 0, flush)
    copies = inp.extra[0]
    alg = copies * (4 * m.n_layers * m.n_heads * m.head_dim * 2 + 16 + 2 * m.rotary_dim * 4)
    del pool
    torch.cuda.empty_cache()
    return {
        "workload": f"gpt-oss-120b 6-turn trajectory, {n} tokens, one prefill",
        "kept": int(keep.sum()), "occurrences": window.occurrence_count, "segments": window.segment_count,
        "copies": copies,
        "host_layout_compile_ms": round((t1 - t0) * 1e3, 2), "host_window_compile_ms": round((t2 - t1) * 1e3, 2),
        "host_pack_ms": round((t3 - t2) * 1e3, 2),
        "bind_ms_back_to_back": round(warm_bind, 5), "bind_p50_ms": round(percentile(cold_bind, 50), 5),
        "reposition_ms": round(warm_repo, 4),
        "reposition_pct_hbm_peak": round(100 * alg / (warm_repo / 1e3) / 1e9 / HBM_PEAK_GBS, 2),
        "kernel_launches": {"bind": 2, "reposition": 1},
    }


CHUNKS = 4


def _published_terminals(state, layout, query_end):
    """Raw tokens [0, query_end) whose terminal versions the forward ending at
    query_end binds (the scheduler's choice, an input of the plan): kept
    tokens that have an owner to bind from -- every token new in this
    forward does, an earlier one needs a canonical or terminal row -- and,
    before the last forward, only those already at their final position."""
    start = len(state.canonical_rows)
    final = np.asarray(layout.positions[:query_end])
    kept = np.asarray(layout.keep_mask[:query_end], dtype=bool)
    terminal = state.terminal_rows.numpy() >= 0
    owner = np.concatenate(((state.canonical_rows.numpy() >= 0) | terminal, np.ones(query_end - start, bool)))
    if query_end == len(layout.positions):
        return torch.from_numpy(kept & owner)
    ready = np.concatenate(((state.canonical_positions.numpy() == final[:start]) | terminal,
                            np.asarray(layout.birth_positions[start:query_end]) == final[start:]))
    return torch.from_numpy(kept & owner & ready)


def _chunked_lifecycle(device, lay, visible, n, chunks, slot_perm, on_copies=None, timings=None):
    """One request prefilled in ``chunks`` forwards: window (C++), plan
    (C++), slot allocation, advance (C++ + one gather launch), the chunk's
    Reposition (``on_copies``).  Returns the final state."""
    from akv_amd import occurrence as ow
    from akv_amd import ownership as own

    state = own.OccurrenceState.empty(device)
    next_slot = 0
    bounds = np.linspace(0, n, chunks + 1).astype(int)
    for qs, qe in zip(bounds[:-1], bounds[1:]):
        t0 = time.perf_counter()
        window = ow.compile_occurrence_window(lay, visible, lay.positions, query_start=int(qs), query_end=int(qe))
        t1 = time.perf_counter()
        plan = state.plan(window, _published_terminals(state, lay, int(qe)))
        t2 = time.perf_counter()
        q = slot_perm[next_slot : next_slot + qe - qs]
        extra = slot_perm[next_slot + qe - qs : next_slot + qe - qs + plan.extra_page_count]
        next_slot += qe - qs + plan.extra_page_count
        adv = state.advance(window, plan, q, extra, visible)
        t3 = time.perf_counter()
        if on_copies is not None:
            on_copies(adv)
        state = adv.state
        if timings is not None:
            timings.append(dict(window=t1 - t0, plan=t2 - t1, advance=t3 - t2, copies=int(plan.extra_page_count),
                                occurrences=window.occurrence_count))
    return state


def chunked_config(device, flush):
    """The same 6-turn 32768-token trajectory prefilled in 4 chunks of 8192
    (chunked prefill): per chunk the host window / plan / advance (C++), one
    gather launch for every slot list of the forward and the Reposition of
    its copies."""
    from akv_amd import plan as lp

    n = 32768
    events, visible = synth.trajectory_events(n, 6, 500, 2000, seed=6)
    lay = lp.compile_context_layout(**events)
    m = synth.GPT_OSS_120B
    pool_slots = 3 * n
    rng = np.random.default_rng(7)
    perm = torch.from_numpy(rng.permutation(np.arange(1, pool_slots)).astype(np.int64)).to(device)
    pool = synth.make_pool(m, pool_slots, device, seed=7, generate_on_device=True)
    w = synth.Workload("trajectory", m, (n,), ((),), 6, 2 * n, pool_slots)
    rope = synth.rope_table(w, device)
    repo_ms, copies = [], []

    def reposition(adv):
        if len(adv.copy_source_slots):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            ops.reposition_kv_layers(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.v[0], adv.copy_source_slots,
                                     adv.copy_destination_slots, adv.copy_position_pairs, rope)
            e.record()
            repo_ms.append((s, e))
            copies.append(len(adv.copy_source_slots))

    _chunked_lifecycle(device, lay, visible, n, CHUNKS, perm)  # warm-up
    torch.cuda.synchronize()
    runs = []
    for _ in range(5):
        timings = []
        repo_ms.clear()
        copies.clear()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        final = _chunked_lifecycle(device, lay, visible, n, CHUNKS, perm, reposition, timings)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        runs.append((wall, timings, [a.elapsed_time(b) for a, b in repo_ms], list(copies)))
    wall, timings, repo, ncopies = sorted(runs, key=lambda r: r[0])[len(runs) // 2]
    term = final.terminal_slots()
    kept = int((term >= 0).sum())
    alg = sum(ncopies) * (4 * m.n_layers * m.n_heads * m.head_dim * 2 + 16 + 2 * m.rotary_dim * 4)
    del pool
    torch.cuda.empty_cache()
    ms = lambda key: [round(t[key] * 1e3, 3) for t in timings]
    return {
        "workload": f"gpt-oss-120b 6-turn trajectory, {n} tokens, {CHUNKS} chunked forwards",
        "kept": kept, "copies_per_chunk": ncopies, "occurrences_per_chunk": [t["occurrences"] for t in timings],
        "host_window_ms": ms("window"), "host_plan_ms": ms("plan"), "advance_ms": ms("advance"),
        "reposition_ms": [round(x, 4) for x in repo],
        "reposition_pct_hbm_peak": round(100 * alg / (sum(repo) / 1e3) / 1e9 / HBM_PEAK_GBS, 2) if repo else None,
        "request_wall_ms": round(wall * 1e3, 2),
        "kernel_launches_per_chunk": {"advance gather": 1, "reposition": 1},
    }


def handoff_config(device, flush):
    """Compacted final-version handoff of the 32k GPT-OSS request: its 19441
    active rows x 36 layers (K and V) packed into a contiguous buffer (P
    side), unpacked into fresh owners of a second pool (D side), and copied
    pool to pool directly (the single-GPU stand-in for peer writes)."""
    from akv_amd import transfer

    m = synth.GPT_OSS_120B
    w = synth.workload("gpt-oss-32k")
    kept = int(synth.compile_layouts(w)[0].keep_mask.sum())
    rng = np.random.default_rng(8)
    src_pool = synth.make_pool(m, w.pool_slots, device, seed=8, generate_on_device=True)
    dst_pool = synth.make_pool(m, w.pool_slots, device, seed=9, generate_on_device=True)
    active = torch.from_numpy(rng.choice(np.arange(1, w.pool_slots), kept, replace=False).astype(np.int32)).to(device)
    owners = torch.from_numpy(rng.choice(np.arange(1, w.pool_slots), kept, replace=False).astype(np.int32)).to(device)
    packed = transfer.PackedKV.empty(m.n_layers, kept, m.n_heads, m.head_dim, m.dtype, device)

    def pack():
        transfer.pack_active_kv(src_pool.k_ptrs, src_pool.v_ptrs, src_pool.k[0], active, packed)

    def unpack():
        transfer.unpack_active_kv(packed, dst_pool.k_ptrs, dst_pool.v_ptrs, dst_pool.k[0], owners)

    def direct():
        transfer.copy_kv_rows(src_pool.k_ptrs, src_pool.v_ptrs, src_pool.k[0], dst_pool.k_ptrs, dst_pool.v_ptrs,
                              dst_pool.k[0], kept, src_slots=active, dst_slots=owners)

    moved = kept * m.n_layers * 2 * m.n_heads * m.head_dim * 2 * 2  # read + write
    out = {"workload": f"{w.name} active rows ({kept} tokens x {m.n_layers} layers, K and V)",
           "bytes_per_copy": moved}
    for name, fn in (("pack", pack), ("unpack", unpack), ("pool_to_pool", direct)):
        warm, _ = _time_steps(fn, 20, 3, 0, flush)
        out[f"{name}_ms"] = round(warm, 4)
        out[f"{name}_pct_hbm_peak"] = round(100 * moved / (warm / 1e3) / 1e9 / HBM_PEAK_GBS, 2)
    del src_pool, dst_pool, packed
    torch.cuda.empty_cache()
    out["kernel_launches_per_copy"] = 1
    return out


def _prefill(device, flush, *, hq, hkv, d, sinks, windows, extend=4096):
    """Next turn's prefill over the compacted 32k request: ``extend`` new
    tokens attend to its 19441 kept tokens (positions with the dropped
    holes) and causally to themselves; one launch per layer kind."""
    from akv_amd import context_attention as ca

    w = synth.workload("gpt-oss-32k")
    lay = synth.compile_layouts(w)[0]
    keep = np.asarray(lay.keep_mask)
    kept_pos = np.asarray(lay.positions)[keep].astype(np.int64)
    plen = len(kept_pos)
    nxt = int(lay.next_position)
    qpos = np.arange(nxt, nxt + extend, dtype=np.int64)
    slots = 2 * plen + 1
    g = torch.Generator(device=device)
    g.manual_seed(11)
    q = torch.randn((extend, hq, d), generator=g, device=device).to(torch.bfloat16)
    ke = torch.randn((extend, hkv, d), generator=g, device=device).to(torch.bfloat16)
    ve = torch.randn((extend, hkv, d), generator=g, device=device).to(torch.bfloat16)
    kp = torch.randn((slots, hkv, d), generator=g, device=device).to(torch.bfloat16)
    vp = torch.randn((slots, hkv, d), generator=g, device=device).to(torch.bfloat16)
    sink_t = torch.randn(hq, generator=g, device=device) if sinks else None
    rng = np.random.default_rng(11)
    idx = torch.from_numpy(rng.permutation(np.arange(1, slots))[:plen].astype(np.int32)).to(device)
    qo = torch.tensor([0, extend], dtype=torch.int64, device=device)
    kv = torch.tensor([0, plen], dtype=torch.int64, device=device)
    qp = torch.from_numpy(qpos).to(device)
    kpp = torch.from_numpy(kept_pos).to(device)
    out = torch.empty_like(q)

    def layer(window):
        return lambda: ca.extend_attention_fwd(q, ke, ve, out, kp, vp, qo, kv, idx, None, True, None, extend,
                                               sm_scale=d ** -0.5, sliding_window_size=window, sinks=sink_t,
                                               context_q_positions=qp, context_kv_positions=kpp)

    warm_full, cold_full = _time_steps(layer(-1), 10, 3, 10, flush)
    # causal flops: QK^T and PV, 2 flops per multiply-add each
    flops_full = 4 * hq * d * sum(plen + i + 1 for i in range(extend))
    r = {
        "full_layer_ms": round(warm_full, 4), "full_layer_p50_ms": round(percentile(cold_full, 50), 4),
        "full_layer_TFLOPs": round(flops_full / (warm_full / 1e3) / 1e12, 1),
        "full_layer_pct_mfma_bf16_peak": round(100 * flops_full / (warm_full / 1e3) / 2.5e15, 2),
    }
    for window in windows:
        warm_win, cold_win = _time_steps(layer(window), 20, 3, 10, flush)
        r[f"window{window}_layer_ms"] = round(warm_win, 4)
        r[f"window{window}_layer_p50_ms"] = round(percentile(cold_win, 50), 4)
    r["kernel_launches_per_layer"] = 1
    return r, plen


def prefill_config(device, flush, extend=4096):
    """GPT-OSS layers (64 q / 8 KV heads x 64, sinks): a full layer and a
    128-window layer."""
    r, plen = _prefill(device, flush, hq=64, hkv=8, d=64, sinks=True, windows=(128,), extend=extend)
    return {"workload": f"gpt-oss-120b prefill of {extend} tokens over {plen} kept tokens "
                        f"(64 q / 8 KV heads x 64, sinks)", **r}


def prefill_llama_config(device, flush, extend=4096):
    """Llama-3-8B layer shape (32 q / 8 KV heads x 128, no sinks, no window)
    over the same request metadata."""
    r, plen = _prefill(device, flush, hq=32, hkv=8, d=128, sinks=False, windows=(), extend=extend)
    return {"workload": f"llama3-8b prefill of {extend} tokens over {plen} kept tokens (32 q / 8 KV heads x 128)", **r}


CEILING_ROUNDS = 3


def _alternating(legs, steps, warmup, flush):
    """Median launch time of each leg over CEILING_ROUNDS rounds, the legs
    taking turns within every round (none always runs first after other
    work)."""
    times = {name: [] for name in legs}
    for _ in range(CEILING_ROUNDS):
        for name, fn in legs.items():
            times[name].append(_time_steps(fn, steps, warmup, 0, flush)[0])
    return {name: float(np.median(v)) for name, v in times.items()}


def _torch_rows_legs(pipe, steps, warmup, flush):
    """The moved K/V rows through kernels not written here: torch's
    index_select (rows gathered into a packed tensor) and index_copy_
    (scattered back), over one int16 [2 x layers, slots, row] tensor so that
    each is a single launch over every layer.  Rates count the rows' bytes
    read and written by each launch."""
    m, o = pipe.w.model, pipe.out
    n, layers = pipe.moved, 2 * m.n_layers
    row = m.n_heads * m.head_dim
    big = torch.empty((layers, pipe.w.pool_slots, row), dtype=torch.int16, device=pipe.device)
    big.random_(-1000, 1000)
    src, dst = o.copy_src.long(), o.copy_dst.long()
    tmp = torch.empty((layers, n, row), dtype=torch.int16, device=pipe.device)
    nbytes = 2 * n * layers * row * 2
    ms = _alternating({"select": lambda: torch.index_select(big, 1, src, out=tmp),
                       "copy": lambda: big.index_copy_(1, dst, tmp)}, steps, warmup, flush)
    del big, tmp
    torch.cuda.empty_cache()
    return {"index_select_GBs": round(nbytes / (ms["select"] / 1e3) / 1e9, 1),
            "index_copy_GBs": round(nbytes / (ms["copy"] / 1e3) / 1e9, 1)}


def _gather_legs(pipe, steps, warmup, flush, orders):
    """akv_copy_kv_rows of the pipeline's src -> dst rows beside its
    Reposition, in the given list orders (the Reposition's output does not
    depend on the order: destinations are disjoint)."""
    from akv_amd import transfer

    o, p, m = pipe.out, pipe.pool, pipe.w.model
    n = pipe.moved
    out = {"gather_copy_GBs": {}, "reposition_GBs": {}}
    for name, perm in orders.items():
        src = o.copy_src if perm is None else o.copy_src[perm].contiguous()
        dst = o.copy_dst if perm is None else o.copy_dst[perm].contiguous()
        pairs = o.copy_pairs if perm is None else o.copy_pairs[perm].contiguous()

        def gather():
            transfer.copy_kv_rows(p.k_ptrs, p.v_ptrs, p.k[0], p.k_ptrs, p.v_ptrs, p.k[0], n, src_slots=src,
                                  dst_slots=dst)

        def repo():
            ops.reposition_kv_layers(p.k_ptrs, p.v_ptrs, p.k[0], p.v[0], src, dst, pairs, pipe.rope,
                                     is_neox_style=m.is_neox_style)

        ms = _alternating({"gather": gather, "repo": repo}, steps, warmup, flush)
        out["gather_copy_GBs"][name] = round(pipe.retained_bytes / (ms["gather"] / 1e3) / 1e9, 1)
        out["reposition_GBs"][name] = round(pipe.alg_bytes / (ms["repo"] / 1e3) / 1e9, 1)
    return out


def _streaming_leg(pipe, steps, warmup, flush):
    from akv_amd import transfer

    m, n = pipe.w.model, pipe.moved
    a = transfer.PackedKV.empty(m.n_layers, n, m.n_heads, m.head_dim, m.dtype, pipe.device)
    b = transfer.PackedKV.empty(m.n_layers, n, m.n_heads, m.head_dim, m.dtype, pipe.device)
    a.k.fill_(1.0)
    a.v.fill_(1.0)
    warm, _ = _time_steps(lambda: transfer.copy_kv_rows(a.k_ptrs, a.v_ptrs, a.k[0], b.k_ptrs, b.v_ptrs, b.k[0], n),
                          steps, warmup, 0, flush)
    del a, b
    torch.cuda.empty_cache()
    return round(pipe.retained_bytes / (warm / 1e3) / 1e9, 1)


def _row_size_legs(pipe, steps, warmup, flush):
    """The same random src -> dst lists over pools of 4 and 16 KV heads
    (512 B and 2 KiB rows): does the random pattern's ceiling move with the
    row size?"""
    import dataclasses

    from akv_amd import transfer

    o, m, n = pipe.out, pipe.w.model, pipe.moved
    out = {}
    for heads in (4, 16):
        model = dataclasses.replace(m, n_heads=heads)
        pool = synth.make_pool(model, pipe.w.pool_slots, pipe.device, seed=3, generate_on_device=True)
        nbytes = n * 4 * m.n_layers * heads * m.head_dim * 2
        warm, _ = _time_steps(lambda: transfer.copy_kv_rows(pool.k_ptrs, pool.v_ptrs, pool.k[0], pool.k_ptrs,
                                                            pool.v_ptrs, pool.k[0], n, src_slots=o.copy_src,
                                                            dst_slots=o.copy_dst), steps, warmup, 0, flush)
        out[f"{heads * m.head_dim * 2}B"] = round(nbytes / (warm / 1e3) / 1e9, 1)
        del pool
        torch.cuda.empty_cache()
    return out


def ceiling_legs(pipe, steps, warmup, flush):
    """Ceilings of the Reposition's access pattern, timed in the same run.

    Random slots (the workload's own lists):
    * gather copy: ``akv_copy_kv_rows`` of the same source -> destination K
      and V rows of every layer (no arithmetic, one launch, stores
      nontemporal like the Reposition's), in raw order,
      sorted by source slot and sorted by destination slot, each beside the
      Reposition with its lists in the same order;
    * torch's ``index_select`` / ``index_copy_`` over the same rows (kernels
      not written here);
    * the gather at 512 B and 2 KiB rows (the same lists over 4- and 16-head
      pools);
    * streaming copy: the same byte count between two packed buffers.
    Ascending slots (the same request, slots from an unfragmented free list):
    the gather, the Reposition, torch's pair and the streaming copy.
    Rates: K/V bytes read + written per launch / average launch time; the
    Reposition's rate counts its algorithmic bytes (slot lists and table rows
    as well), as ``roofline.achieved`` does."""
    o = pipe.out
    orders = {"raw": None, "by_source_slot": torch.argsort(o.copy_src), "by_destination_slot": torch.argsort(o.copy_dst)}
    out = {"random": _gather_legs(pipe, steps, warmup, flush, orders)}
    r = out["random"]
    r["torch"] = _torch_rows_legs(pipe, steps, warmup, flush)
    r["gather_copy_by_row_size_GBs"] = _row_size_legs(pipe, steps, warmup, flush)
    r["streaming_copy_GBs"] = _streaming_leg(pipe, steps, warmup, flush)
    r["reposition_frac_of_gather"] = round(r["reposition_GBs"]["raw"] / r["gather_copy_GBs"]["raw"], 4)
    r["reposition_frac_of_streaming"] = round(r["reposition_GBs"]["raw"] / r["streaming_copy_GBs"], 4)
    asc = Pipeline(pipe.w_name, pipe.device, slot_order="ascending")
    asc.compaction()
    a = out["ascending"] = _gather_legs(asc, steps, warmup, flush, {"raw": None})
    a["torch"] = _torch_rows_legs(asc, steps, warmup, flush)
    a["streaming_copy_GBs"] = _streaming_leg(asc, steps, warmup, flush)
    a["reposition_frac_of_gather"] = round(a["reposition_GBs"]["raw"] / a["gather_copy_GBs"]["raw"], 4)
    del asc
    torch.cuda.empty_cache()
    best = max([v for v in r["gather_copy_GBs"].values()] + list(r["torch"].values())
               + list(r["gather_copy_by_row_size_GBs"].values()))
    out["best_random_row_copy_pct_hbm_peak"] = round(100 * best / HBM_PEAK_GBS, 2)
    out["kernel"] = ("akv_copy_kv_rows (layer-major, one row per wave, nontemporal stores as in the "
                     "Reposition); torch index_select / index_copy_")
    out["rounds"] = CEILING_ROUNDS
    return out


def read_pmc_traffic():
    """HBM bytes per Reposition launch from the committed rocprof PMC summary."""
    if not PMC_SUMMARY.exists():
        return None
    for line in PMC_SUMMARY.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_threads():
    """Host threads the baseline may use: OMP_NUM_THREADS when set (the GPU
    box sets it to its CPU share), else the CPUs this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def cpu_baseline(pipe, runs):
    """The reference path restated on the host CPU, same workload, same run.

    Per run: the Drop + Reposition event compile (``oracle.events``, Python,
    single thread, as the reference's host compiler), the table update /
    freed list / copy lists (``oracle.occurrence``, numpy), the Reposition of
    all moved tokens over all layers (``oracle.cpu_torch``, torch CPU fp32
    vectorised over every host thread) and the decode indices.  Reported:
    p50 over ``runs`` runs; ``value`` = retained-KV bytes / p50 of the
    Reposition alone (the metric's unit), and the whole step's p50 beside it.
    The CPU result of the last run is compared bit for bit with the GPU's
    over every destination row of every layer."""
    from oracle import cpu_torch
    from oracle import events as oe
    from oracle import occurrence as occ

    threads = cpu_threads()
    torch.set_num_threads(threads)
    w, m = pipe.w, pipe.w.model
    ev = {k: v.numpy() for k, v in synth.request_events(pipe.n, w.spans[0]).items()}
    # the GPU result at every destination row, then host copies of the pool
    pipe.reposition()
    torch.cuda.synchronize()
    dst = pipe.out.copy_dst.long()
    gpu_k = [t[dst].cpu() for t in pipe.pool.k]
    gpu_v = [t[dst].cpu() for t in pipe.pool.v]
    host_k = [t.cpu() for t in pipe.pool.k]
    host_v = [t.cpu() for t in pipe.pool.v]
    table = pipe.rope.cpu()
    step_s, repo_s = [], []
    for _ in range(runs):
        t0 = time.perf_counter()
        lay = oe.compile_context_layout(*(ev[k] for k in ("token_ids", "drop_insert_offsets", "drop_range_offsets",
                                                          "drop_ranges", "reposition_raw_boundaries",
                                                          "reposition_insert_offsets")))
        cf = occ.closed_form(pipe.slots.birth_rows[0], lay.keep_mask, lay.birth_positions, lay.positions,
                             pipe.slots.fresh[0])
        t1 = time.perf_counter()
        cpu_torch.reposition_kv_layers(host_k, host_v, cf["copy_source_slots"], cf["copy_destination_slots"],
                                       cf["copy_position_pairs"], table, is_neox_style=m.is_neox_style)
        t2 = time.perf_counter()
        np.concatenate((cf["active_slots"], [int(pipe.slots.fresh[0][0])]))  # decode indices, one new token
        t3 = time.perf_counter()
        step_s.append(t3 - t0)
        repo_s.append(t2 - t1)
    cdst = torch.from_numpy(cf["copy_destination_slots"].astype(np.int64))
    exact = bool(torch.equal(cdst, dst.cpu())) and all(
        torch.equal(h[cdst].view(torch.int16), g.view(torch.int16)) for h, g in zip(host_k + host_v, gpu_k + gpu_v))
    del host_k, host_v, gpu_k, gpu_v
    repo_p50 = percentile(repo_s, 50)
    step_p50 = percentile(step_s, 50)
    chunked_s = _chunked_ownership_port()
    return {
        "value": round(pipe.retained_bytes / repo_p50 / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"the whole 32k GPT-OSS request, {runs} runs: Reposition of all {pipe.moved} moved tokens x "
                   f"{m.n_layers} layers in torch CPU fp32 on {threads} threads (oracle.cpu_torch), plus the "
                   f"Python event compile and numpy tables of the same step"),
        "reposition_p50_ms": round(repo_p50 * 1e3, 1),
        "step_p50_ms": round(step_p50 * 1e3, 1),
        "step_value_GBs": round(pipe.retained_bytes / step_p50 / 1e9, 3),
        "runs": runs,
        "bit_exact_vs_gpu": exact,
        "chunked_ownership_ms": round(chunked_s * 1e3, 1),
        "chunked_ownership_sample": (f"numpy oracle of the chunked-prefill ownership (window, plan, advance; "
                                     f"{CHUNKS} chunks of the 32768-token trajectory), host time"),
        "host": host_info(threads),
    }


def _chunked_ownership_port():
    """Host seconds of the numpy oracle over the chunked lifecycle that
    ``chunked_config`` runs natively (slots stay numpy here)."""
    from oracle import events as oe
    from oracle import occurrence as occ
    from oracle import ownership as own

    n = 32768
    events, visible = synth.trajectory_events(n, 6, 500, 2000, seed=6)
    ref = oe.compile_context_layout(*(events[k].numpy() for k in events))
    visible = visible.numpy()
    slots = np.random.default_rng(7).permutation(np.arange(1, 3 * n)).astype(np.int64)
    st = own.State.from_match(np.zeros(0, np.int64), np.zeros(0, np.int32), exact_prefix_len=0)
    bounds = np.linspace(0, n, CHUNKS + 1).astype(int)
    used = 0
    t0 = time.perf_counter()
    for qs, qe in zip(bounds[:-1], bounds[1:]):
        win = occ.compile_window(ref, visible, int(qs), int(qe))
        p = st.plan(win, st.prefill_terminal_keep(ref, int(qe)))
        q = slots[used : used + qe - qs]
        extra = slots[used + qe - qs : used + qe - qs + p["extra_page_count"]]
        used += qe - qs + p["extra_page_count"]
        st = st.advance(win, p, q, extra, visible).state
    return time.perf_counter() - t0


def host_event_compile_ms(w, runs=5):
    """Host time of the native event compile (``compile_context_layout``,
    C++) for the workload's requests: median of ``runs`` warm runs."""
    from akv_amd import plan as lp

    events = [synth.request_events(n, spans) for n, spans in zip(w.lengths, w.spans)]
    for e in events:
        lp.compile_context_layout(**e)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for e in events:
            lp.compile_context_layout(**e)
        times.append(time.perf_counter() - t0)
    return round(float(np.median(times)) * 1e3, 3)


def compaction_passes(inputs):
    """Passes akv_compact_rows makes over this batch on this device: 1 (one
    kernel whose tiles meet at an in-kernel barrier) or 2 (count, scatter)."""
    total = sum(inputs.n_tokens)
    return int(_lib.load().akv_compact_launches(inputs.n_requests, total, total + inputs.n_requests, None))


def compaction_launches(inputs):
    """Kernel launches of akv_compact_rows: two on either path (the one-pass
    kernel and its one-workgroup finishing launch, or count and scatter)."""
    return 2 if compaction_passes(inputs) else 0


def host_info(threads):
    """CPU model and core counts of this host, read from /proc/cpuinfo (no
    child process is started from the GPU process)."""
    fields, physical = {}, set()
    try:
        with open("/proc/cpuinfo") as f:
            block = {}
            for line in f.read().splitlines() + [""]:
                if not line.strip():
                    if block:
                        for key in ("model name", "vendor_id", "cpu family", "model", "stepping"):
                            fields.setdefault(key, block.get(key, ""))
                        physical.add((block.get("physical id", "0"), block.get("core id", block.get("processor"))))
                    block = {}
                    continue
                key, _, val = line.partition(":")
                block[key.strip()] = val.strip()
    except OSError:
        pass
    family = fields.get("cpu family", "?")
    return {"cpu": fields.get("model name", ""),
            "cpu_family_model_stepping": "/".join(fields.get(k, "?") for k in ("cpu family", "model", "stepping")),
            # AMD family 26 (1Ah) is the Zen 5 core of the EPYC 9005 series
            "cpu_core_generation": "Zen 5 (EPYC 9005 series)" if family == "26" and "AMD" in fields.get(
                "vendor_id", "") + fields.get("model name", "") else None,
            "physical_cores": len(physical) or None,
            "logical_cpus": os.cpu_count(), "cpus_available": len(os.sched_getaffinity(0)),
            "torch_threads": threads}


def percentile(xs, q):
    return float(np.percentile(np.asarray(xs), q))


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported here "
              "(the Drop + Reposition path shards by KV head under TP with no communication)", file=sys.stderr)
        raise SystemExit(2)
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.copy_calibration:
        copy_calibration(device)
        return
    if args.only:
        scratch = torch.ones(1 << 28, dtype=torch.float32, device=device)
        sink = torch.empty((), device=device)
        flush = lambda: torch.sum(scratch, 0, out=sink)  # noqa: E731
        run = {"handoff": handoff_config, "prefill": prefill_config, "prefill-llama": prefill_llama_config,
               "chunked": chunked_config, "decode": decode_consumer_config, "ragged": ragged_config}[args.only]
        print(json.dumps(run(device, flush)), flush=True)
        return
    pipe = Pipeline(args.workload, device)
    pipe.compaction()
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        if not args.reposition_only:
            pipe.compaction()
        pipe.reposition()
    torch.cuda.synchronize()
    print(f"# warmup done: {args.warmup} steps", file=sys.stderr, flush=True)

    # throughput: K back-to-back steps; HIP events on the launch stream also
    # bracket every Reposition launch inside the timed region
    repo_events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for before, after in repo_events:
        if not args.reposition_only:
            pipe.compaction()
        before.record()
        pipe.reposition()
        after.record()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = start.elapsed_time(end) / args.steps
    repo_timed_ms = [b.elapsed_time(a) for b, a in repo_events]
    print(f"# timed {args.steps} steps: {ms_per_step:.4f} ms/step (wall {wall_ms:.1f} ms), "
          f"reposition {np.mean(repo_timed_ms):.4f} ms", file=sys.stderr, flush=True)

    # latency with a cold MALL: events around the whole step and the Reposition alone
    step_ms, repo_ms = [], []
    for _ in range(args.latency_iters):
        pipe.flush()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e2 = torch.cuda.Event(enable_timing=True)
        e0.record()
        if not args.reposition_only:
            pipe.compaction()
        e1.record()
        pipe.reposition()
        e2.record()
        torch.cuda.synchronize()
        step_ms.append(e0.elapsed_time(e2))
        repo_ms.append(e1.elapsed_time(e2))
    print(f"# latency iterations done: {args.latency_iters}", file=sys.stderr, flush=True)
    # a check of this run (after every timed step, not between compaction and
    # Reposition): the lists were complete
    status = None if args.reposition_only else tables.check_status(pipe.out)

    # the same launch with every pair at its birth position: a pure row copy
    # of the same slots (same bytes, no rotation) -- the access pattern's own
    # rate, against which the rotation's cost shows
    copy_only = ceiling = None
    if not args.reposition_only:
        o, p, neox = pipe.out, pipe.pool, pipe.w.model.is_neox_style
        same = torch.stack((o.copy_pairs[:, 0], o.copy_pairs[:, 0]), 1).contiguous()

        def copy_step():
            ops.reposition_kv_layers(p.k_ptrs, p.v_ptrs, p.k[0], p.v[0], o.copy_src, o.copy_dst, same, pipe.rope,
                                     is_neox_style=neox)

        warm_copy, _ = _time_steps(copy_step, args.steps, args.warmup, 0, pipe.flush)
        copy_only = {"ms": round(warm_copy, 5),
                     "pct_hbm_peak": round(100 * pipe.alg_bytes / (warm_copy / 1e3) / 1e9 / HBM_PEAK_GBS, 2)}
        print("# ceiling legs ...", file=sys.stderr, flush=True)
        ceiling = ceiling_legs(pipe, args.steps, args.warmup, pipe.flush)

    # roofline of the dominant kernel: its average launch inside the timed
    # (back-to-back, steady-state) region
    repo_avg_s = float(np.mean(repo_timed_ms)) / 1e3
    achieved = pipe.alg_bytes / repo_avg_s / 1e9
    traffic = read_pmc_traffic()
    m = pipe.w.model
    result = {
        "metric": METRIC,
        "value": round(pipe.retained_bytes / (ms_per_step / 1e3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": pipe.w.name,
            "layers": m.n_layers,
            "kv_heads": m.n_heads,
            "head_dim": m.head_dim,
            "kv_dtype": "bf16",
            "rope": "yarn(theta=150000, factor=32, original=4096)",
            "tokens": pipe.n,
            "kept": pipe.kept,
            "moved": pipe.moved,
            "page_size": 1,
            "step": "reposition only" if args.reposition_only else "page-table compaction + reposition",
        },
        # per-iteration latency after a 1 GiB read flush of L2 + MALL
        "p50_ms": round(percentile(step_ms, 50), 5),
        "p99_ms": round(percentile(step_ms, 99), 5),
        "reposition_p50_ms": round(percentile(repo_ms, 50), 5),
        "reposition_p99_ms": round(percentile(repo_ms, 99), 5),
        "reposition_steady_ms": round(float(np.mean(repo_timed_ms)), 5),
        # same slots, pairs at the birth position (a bit copy, no rotation)
        "reposition_copy_only": copy_only,
        # the access pattern's own ceilings, same run (see ceiling_legs)
        "ceiling": ceiling,
        "pct_hbm_peak": round(100 * achieved / HBM_PEAK_GBS, 2),
        # compaction: two launches (one pass + its finishing workgroup);
        # Reposition: one launch for the 36-layer group, gated on the device
        # by the compaction's status word
        "kernel_launches_per_step": 1 if args.reposition_only else compaction_launches(pipe.inputs) + 1,
        "compaction_passes": None if args.reposition_only else compaction_passes(pipe.inputs),
        "compaction_status": status,
        # the request's Drop + Reposition events compiled on the host (C++),
        # median of 5 warm runs: the CPU work before the step's launches
        "host_event_compile_ms": host_event_compile_ms(pipe.w),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "reposition_vec_kernel<bf16, f32, neox>",
            "bytes_per_launch": pipe.alg_bytes,
        },
    }
    if not args.reposition_only:
        print("# secondary configurations ...", file=sys.stderr, flush=True)
        result["other_configs"] = [tiny_config(device, pipe.flush), ascending_slots_config(device, pipe.flush),
                                   median_moved_config(device, pipe.flush), tp2_share_config(device, pipe.flush),
                                   ragged_config(device, pipe.flush), decode_consumer_config(device, pipe.flush),
                                   prefill_config(device, pipe.flush), prefill_llama_config(device, pipe.flush),
                                   multistage_config(device, pipe.flush),
                                   chunked_config(device, pipe.flush), handoff_config(device, pipe.flush)]
        if not args.no_cow:
            print("# copy-on-write configuration ...", file=sys.stderr, flush=True)
            result["other_configs"].append(cow_config(device, pipe.flush))
    if not args.no_cpu_baseline:
        print("# cpu baseline ...", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(pipe, args.cpu_runs)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
