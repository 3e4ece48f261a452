// Batched page-table compaction of a single-owner final forward (gfx950).
//
// For every raw token of every request: kept / moved / retired flags from the
// keep mask and the birth vs final positions, then order-preserving stream
// compaction into the flat outputs.  Semantics: the final-forward result of
// OccurrenceState.advance + terminal_slots
// (akv/system/sglang/srt/context_system/occurrence.py:632-767) written into
// the raw request row (akv/system/sglang.patch:3161-3164), the decode layout
// of ContextDecodeLayout.from_layout (occurrence.py:47-66) and the compacted
// active row of request_active_slots
// (akv/system/sglang/srt/disaggregation/context_transfer.py:110-128).
//
// Two launches over tiles of 256 x STEPS tokens of the concatenated batch
// (STEPS grows until the batch is about 2048 tiles):
//   count    per tile: its kept / moved / retired counts and the generated
//            entries of the requests that start in it (its aggregate); per
//            request: the tile's counts before the request's first token
//            and the request's raw row (two tiles per workgroup);
//   scatter  per tile: its exclusive prefix, summed from every earlier
//            tile's aggregate (16 bytes each, read in one unrolled batch of
//            up to 2304 issued with the tile's own inputs), then every
//            output the tile owns.
// No workgroup waits for another and the workspace needs no clearing.  A
// single-pass scan with decoupled look-back measured slower on this batch:
// per-tile chains of dependent global round trips (publish, poll, read)
// cost ~10 us under load, and 2048 tiles do not all fit on the chip at once.
//
// Loads are unconditional, from indices clamped into range, with the value
// selected afterwards: a load under a divergent condition is followed by a
// wait for every load in flight, which serialises the tile.  Batches of up
// to 512 requests keep their offsets, generated counts and rows in LDS
// (STAGED); larger ones read them from memory.
#include "common.h"

// Wavefront reduce / scan of the device library (DPP and lane reads, no
// LDS); every lane of the wave must be active.
extern "C" __device__ long long __ockl_wfred_add_i64(long long);
extern "C" __device__ long long __ockl_wfscan_add_i64(long long, bool inclusive);
extern "C" __device__ int __ockl_wfscan_add_i32(int, bool inclusive);

namespace akv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSteps = 4;  // at most 1024 tokens per tile
constexpr int64_t kTargetTiles = 2048;
constexpr int kWindow = 256;          // requests per tile held in LDS
constexpr int kStagedRequests = 512;  // batches up to this many requests: offsets in LDS
constexpr int kCounters = 4;          // kept, moved, retired, generated
constexpr int kAggUnroll = 9;         // earlier aggregates per thread per batch
constexpr int kSuper = 2;             // tiles per workgroup of the count launch

int tile_steps(int64_t total) {
  int steps = 1;
  while (steps < kMaxSteps && total > static_cast<int64_t>(kThreads) * steps * kTargetTiles) steps <<= 1;
  return steps;
}

int64_t tile_count(int64_t total, int steps) {
  const int64_t tile = static_cast<int64_t>(kThreads) * steps;
  return total <= 0 ? 1 : (total + tile - 1) / tile;
}

struct CompactArgs {
  const int64_t* req_offsets;
  int32_t* table;
  int64_t row_stride;
  const int64_t* row_pointers;
  const int64_t* req_rows;
  const uint8_t* keep;
  const int32_t* birth;
  const int32_t* final_pos;
  const int32_t* birth_slots;  // flat birth slots, or nullptr: read the row
  const int32_t* fresh;  // never null: a dummy word of the workspace when empty
  int64_t fresh_count;
  int32_t* retired;
  int64_t retired_capacity;
  int32_t* copy_src;
  int32_t* copy_dst;
  int32_t* copy_pairs;
  int32_t* raw_indices;
  int32_t* active_positions;
  int64_t kept_capacity;
  const int32_t* generated;
  int32_t* kv_indices;
  int64_t kv_capacity;
  int32_t* kv_indptr;
  int32_t* last_page_len;
  int32_t page_size;
  int32_t* counts;
  int32_t* status;
  int4* tile_agg;      // [tiles] per-tile aggregates (kept, moved, retired, generated)
  int64_t* req_gen;    // [B + 1] generated prefix: of every request (staged batches, count
                       // launch), of the tile's requests (others, tiles with more
                       // requests than the window)
  int32_t** req_row;   // [B] raw row of each request (batches that are not staged)
  int64_t total;       // raw tokens of the batch (req_offsets[B])
  int64_t tiles;
  int32_t n_requests;
};

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// number of set lanes below this one in a 64-bit ballot
__device__ __forceinline__ int rank_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

__device__ __forceinline__ int32_t* row_base(const CompactArgs& a, int64_t b) {
  const int64_t r = a.req_rows[b];
  if (a.row_pointers) return reinterpret_cast<int32_t*>(a.row_pointers[r]);
  return a.table + r * a.row_stride;
}

// Number of entries of the sorted at(0 .. n-1) that are <= x, computed by
// one whole wave (every lane gets the result): each round probes 64 evenly
// spaced entries of the remaining window, one load per lane.
template <typename At>
__device__ int64_t wave_count_le(int64_t n, int64_t x, At at) {
  int64_t lo = 0, len = n;  // entries before lo are <= x; the answer is in [lo, lo + len]
  while (len > 64) {
    const int64_t stride = (len + 63) / 64;
    const int64_t p = lo + lane_id() * stride;
    const bool in = p < lo + len;
    const int64_t v = at(in ? p : lo);
    const int c = __popcll(__ballot(in & (v <= x)));
    if (c == 0) return lo;
    const int64_t first = lo + (c - 1) * stride + 1;
    const int64_t end = lo + c * stride < lo + len ? lo + c * stride : lo + len;
    lo = first;
    len = end - first;
  }
  if (len == 0) return lo;
  const bool in = lane_id() < len;
  const int64_t v = at(in ? lo + lane_id() : lo);
  return lo + __popcll(__ballot(in & (v <= x)));
}

// Workgroup-wide exclusive scan of one int64 per thread: (prefix, total).
__device__ void block_scan(int64_t v, int64_t* lds, int64_t& prefix, int64_t& total) {
  const int64_t inc = __ockl_wfscan_add_i64(v, true);
  const int w = threadIdx.x >> 6;
  if (lane_id() == 63) lds[w] = inc;
  __syncthreads();
  prefix = inc - v;
  total = 0;
  for (int q = 0; q < kWaves; ++q) {
    if (q < w) prefix += lds[q];
    total += lds[q];
  }
  __syncthreads();
}

// Workgroup-wide sums of N int64 per thread (every thread gets them).
template <int N>
__device__ void block_sums(int64_t (&v)[N], int64_t (*lds)[N]) {
#pragma unroll
  for (int c = 0; c < N; ++c) v[c] = __ockl_wfred_add_i64(v[c]);
  if (lane_id() == 0)
#pragma unroll
    for (int c = 0; c < N; ++c) lds[threadIdx.x >> 6][c] = v[c];
  __syncthreads();
#pragma unroll
  for (int c = 0; c < N; ++c) {
    v[c] = 0;
    for (int q = 0; q < kWaves; ++q) v[c] += lds[q][c];
  }
  __syncthreads();
}

// The tile's per-64-token masks and their exclusive counts, in LDS.
template <int BLKS>
struct TileMasks {
  uint64_t bits[BLKS][3];
  int32_t before[BLKS + 1][3];  // before[BLKS] = the tile's totals

  // tokens of counter c among the first q tokens of the tile, q in [0, BLKS * 64]
  __device__ int32_t count_before(int64_t q, int c) const {
    const int blk = static_cast<int>(q >> 6);
    if (blk >= BLKS) return before[BLKS][c];
    const int r = static_cast<int>(q & 63);
    return before[blk][c] + (r ? __popcll(bits[blk][c] & (~0ull >> (64 - r))) : 0);
  }
};

// LDS of both launches: the staged request arrays (STAGED batches), the
// search results and the tile's masks.
template <int STEPS, bool STAGED>
struct Tile {
  static constexpr int kTile = kThreads * STEPS;
  static constexpr int kBlks = kTile / 64;
  static constexpr int kStage = STAGED ? kStagedRequests : 1;
  int64_t s_off[kStage + 1];
  int64_t s_genx[kStage + 1];  // exclusive prefix of generated entries
  int64_t s_rr[kStage];        // request table row of each request
  int64_t s_count[kWaves];
  TileMasks<kBlks> m;
  int64_t lds[kWaves];
};

// Access to request offsets, generated counts and rows.  STAGED: from LDS
// (offsets, the generated prefix the count launch wrote, table rows);
// otherwise from memory (rows the count launch resolved).
template <int STEPS, bool STAGED>
struct Requests {
  const CompactArgs& a;
  const Tile<STEPS, STAGED>& sh;
  __device__ __forceinline__ int64_t off(int64_t b) const {
    if constexpr (STAGED)
      return sh.s_off[b];
    else
      return a.req_offsets[b];
  }
  __device__ __forceinline__ int64_t gen(int64_t b) const {
    if (b >= a.n_requests) return 0;
    if constexpr (STAGED)
      return sh.s_genx[b + 1] - sh.s_genx[b];
    else
      return a.generated ? a.generated[b] : 0;
  }
  __device__ __forceinline__ int32_t* row(int64_t b) const {
    if constexpr (STAGED) {
      const int64_t r = sh.s_rr[b];
      return a.row_pointers ? reinterpret_cast<int32_t*>(a.row_pointers[r]) : a.table + r * a.row_stride;
    } else {
      return a.req_row[b];
    }
  }
};

// One round of loads into LDS: offsets, the generated prefix and table rows.
template <int STEPS, bool STAGED>
__device__ void stage_requests(const CompactArgs& a, Tile<STEPS, STAGED>& sh) {
  if constexpr (STAGED) {
    const int n_off = a.n_requests + 1;
    for (int i = threadIdx.x; i < n_off; i += kThreads) {
      const int ic = i < a.n_requests ? i : a.n_requests - 1;
      const int64_t o = a.req_offsets[i];
      const int64_t g = a.req_gen[i];
      const int64_t r = a.req_rows[ic];
      sh.s_off[i] = o;
      sh.s_genx[i] = g;
      if (i < a.n_requests) sh.s_rr[i] = r;
    }
  }
}

// The tile's keep mask and positions; lanes past t1 read token t1 - 1 (every
// use masks them out, so no select here holds up the next loads).
template <int STEPS>
__device__ __forceinline__ void load_inputs(const CompactArgs& a, int64_t t0, int64_t t1, uint8_t (&kb)[STEPS],
                                            int32_t (&bps)[STEPS], int32_t (&fps)[STEPS]) {
#pragma unroll
  for (int s = 0; s < STEPS; ++s) kb[s] = bps[s] = fps[s] = 0;
  if (t1 <= t0) return;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int64_t t = t0 + s * kThreads + threadIdx.x;
    const int64_t tc = t < t1 ? t : t1 - 1;
    kb[s] = a.keep[tc];
    bps[s] = a.birth[tc];
    fps[s] = a.final_pos[tc];
  }
}

// Searches (wave w: offsets <= x[w]) and the tile's masks and block counts.
// Starts with a barrier, so LDS state of an earlier tile may be reused.
template <int STEPS, bool STAGED>
__device__ void tile_masks(const CompactArgs& a, Tile<STEPS, STAGED>& sh, int64_t t0, int64_t t1,
                           const int64_t (&x)[kWaves], const uint8_t (&kb)[STEPS], const int32_t (&bps)[STEPS],
                           const int32_t (&fps)[STEPS]) {
  const int w = threadIdx.x >> 6;
  __syncthreads();
  const Requests<STEPS, STAGED> rq{a, sh};
  const int64_t c =
      wave_count_le(static_cast<int64_t>(a.n_requests) + 1, x[w], [&](int64_t i) { return rq.off(i); });
  if (lane_id() == 0) sh.s_count[w] = c;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int64_t t = t0 + s * kThreads + threadIdx.x;
    const bool valid = t < t1;
    const bool kept = valid && kb[s] != 0;
    const bool moved = kept && bps[s] != fps[s];
    const bool retired = valid && (!kept || moved);
    const uint64_t mk = __ballot(kept), mm = __ballot(moved), mr = __ballot(retired);
    if (lane_id() < 3) sh.m.bits[s * kWaves + w][lane_id()] = lane_id() == 0 ? mk : (lane_id() == 1 ? mm : mr);
  }
  __syncthreads();
  // exclusive counts per block: lane p of wave 0 scans block p's popcounts
  // (lane kBlks gets the tile's totals)
  if (w == 0) {
    constexpr int kBlks = Tile<STEPS, STAGED>::kBlks;
    const int p = lane_id();
    const int pc = p < kBlks ? p : 0;
#pragma unroll
    for (int cc = 0; cc < 3; ++cc) {
      const int n = __popcll(sh.m.bits[pc][cc]);
      const int ex = __ockl_wfscan_add_i32(p < kBlks ? n : 0, false);
      if (p <= kBlks) sh.m.before[p][cc] = ex;
    }
  }
}

// Per tile (kSuper consecutive tiles per workgroup, inputs loaded up front):
// its kept / moved / retired counts.  Batches of more than kStagedRequests
// requests also get the generated entries of the requests that start in
// the tile and each such request's raw row; smaller ones instead get the
// request-level generated prefix, written by workgroup 0.
template <int STEPS, bool STAGED>
__global__ void __launch_bounds__(kThreads) count_kernel(const CompactArgs a) {
  constexpr int64_t kTile = Tile<STEPS, STAGED>::kTile;
  const int w = threadIdx.x >> 6;
  uint8_t kb[kSuper][STEPS];
  int32_t bps[kSuper][STEPS], fps[kSuper][STEPS];
#pragma unroll
  for (int u = 0; u < kSuper; ++u) {
    const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kSuper + u) * kTile;
    const int64_t t1 = t0 + kTile < a.total ? t0 + kTile : a.total;
    load_inputs<STEPS>(a, t0, t1, kb[u], bps[u], fps[u]);
  }
  __shared__ int64_t lds[kWaves];
  if constexpr (STAGED) {
    if (blockIdx.x == 0) {
      // exclusive prefix of generated entries over requests 0 .. B
      int64_t carry = 0;
      for (int base = 0; base <= a.n_requests; base += kThreads) {
        const int b = base + threadIdx.x;
        const int64_t g = (a.generated && b < a.n_requests) ? a.generated[b] : 0;
        int64_t pre, sum;
        block_scan(g, lds, pre, sum);
        if (b <= a.n_requests) a.req_gen[b] = carry + pre;
        carry += sum;
      }
    }
  }
  // per wave and tile: kept, moved, retired tokens
  __shared__ int32_t red[kSuper][kWaves][3];
#pragma unroll
  for (int u = 0; u < kSuper; ++u) {
    const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kSuper + u) * kTile;
    const int64_t t1 = t0 + kTile < a.total ? t0 + kTile : a.total;
    int32_t n[3] = {0, 0, 0};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const bool valid = t0 + s * kThreads + threadIdx.x < t1;
      const bool kept = valid && kb[u][s] != 0;
      const bool moved = kept && bps[u][s] != fps[u][s];
      const bool retired = valid && (!kept || moved);
      n[0] += __popcll(__ballot(kept));
      n[1] += __popcll(__ballot(moved));
      n[2] += __popcll(__ballot(retired));
    }
    if (lane_id() == 0)
#pragma unroll
      for (int c = 0; c < 3; ++c) red[u][w][c] = n[c];
  }
  __shared__ int32_t gen_own[kSuper];
  if (threadIdx.x < kSuper) gen_own[threadIdx.x] = 0;
  if constexpr (!STAGED) {
    // requests that start in each tile (the last tile also at t1): their
    // generated entries and raw rows
    __shared__ int64_t s_count[kSuper][2];
#pragma unroll
    for (int u = 0; u < kSuper; ++u) {
      const int64_t tile = static_cast<int64_t>(blockIdx.x) * kSuper + u;
      const int64_t t0 = tile * kTile;
      const int64_t t1 = t0 + kTile < a.total ? t0 + kTile : a.total;
      if (w < 2) {
        const int64_t c = wave_count_le(static_cast<int64_t>(a.n_requests) + 1, w == 0 ? t0 - 1 : t1 - 1,
                                        [&](int64_t i) { return a.req_offsets[i]; });
        if (lane_id() == 0) s_count[u][w] = c;
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kSuper; ++u) {
      const int64_t tile = static_cast<int64_t>(blockIdx.x) * kSuper + u;
      if (tile >= a.tiles) break;
      const int64_t own_lo = s_count[u][0];
      const int64_t own_hi = tile == a.tiles - 1 ? static_cast<int64_t>(a.n_requests) : s_count[u][1];
      int64_t g[1] = {0};
      for (int64_t b = own_lo + threadIdx.x; b < own_hi; b += kThreads) {
        g[0] += a.generated ? a.generated[b] : 0;
        a.req_row[b] = row_base(a, b);
      }
      __shared__ int64_t red_g[kWaves][1];
      block_sums<1>(g, red_g);
      // generated entries fit int32 whenever kv_indptr (int32) does
      if (threadIdx.x == 0) gen_own[u] = static_cast<int32_t>(g[0]);
    }
  }
  __syncthreads();
  if (threadIdx.x < kSuper) {
    const int u = threadIdx.x;
    const int64_t tile = static_cast<int64_t>(blockIdx.x) * kSuper + u;
    if (tile < a.tiles) {
      int32_t n[3] = {0, 0, 0};
      for (int q = 0; q < kWaves; ++q)
#pragma unroll
        for (int c = 0; c < 3; ++c) n[c] += red[u][q][c];
      a.tile_agg[tile] = make_int4(n[0], n[1], n[2], gen_own[u]);
    }
  }
}

// Writes one token's outputs: its terminal slot into the raw row and, by
// its ranks among the batch's kept / moved / retired tokens, the lists.
__device__ __forceinline__ void emit_token(const CompactArgs& a, bool kept, int32_t bpos, int32_t fpos, int32_t slot,
                                           int32_t fresh, int64_t pk, int64_t pm, int64_t pr, int32_t* row,
                                           int64_t local, int64_t shift) {
  const bool moved = kept && bpos != fpos;
  const bool retired = !kept || moved;
  int32_t terminal = -1;
  if (moved) {
    terminal = fresh;
    if (pm < a.fresh_count) {
      a.copy_src[pm] = slot;
      a.copy_dst[pm] = fresh;
      a.copy_pairs[2 * pm] = bpos;
      a.copy_pairs[2 * pm + 1] = fpos;
    }
  } else if (kept) {
    terminal = slot;
  }
  if (retired && pr < a.retired_capacity) a.retired[pr] = slot;
  if (kept && pk < a.kept_capacity) {
    a.raw_indices[pk] = static_cast<int32_t>(local);
    a.active_positions[pk] = fpos;
  }
  if (kept && a.kv_indices && pk + shift < a.kv_capacity) a.kv_indices[pk + shift] = terminal;
  row[local] = terminal;
}

// Per tile: the exclusive prefix, then every output the tile owns.
template <int STEPS, bool STAGED>
__global__ void __launch_bounds__(kThreads) scatter_kernel(const CompactArgs a) {
  using T = Tile<STEPS, STAGED>;
  __shared__ T sh;
  const int w = threadIdx.x >> 6;
  const int64_t tile = blockIdx.x;
  const bool last_tile = tile == a.tiles - 1;
  const int64_t t0 = tile * T::kTile;
  const int64_t t1 = t0 + T::kTile < a.total ? t0 + T::kTile : a.total;
  // aggregates of earlier tiles: the first batch in flight with the inputs
  int4 agg[kAggUnroll];
#pragma unroll
  for (int u = 0; u < kAggUnroll; ++u) {
    const int64_t i = u * kThreads + threadIdx.x;
    agg[u] = a.tile_agg[i < tile ? i : 0];
  }
  uint8_t kb[STEPS];
  int32_t bps[STEPS], fps[STEPS];
  load_inputs<STEPS>(a, t0, t1, kb, bps, fps);
  stage_requests<STEPS, STAGED>(a, sh);
  // this thread's share of the exclusive prefix: kept, moved, retired and
  // (batches that are not staged) generated entries before the tile
  int64_t sums[kCounters] = {0, 0, 0, 0};
  for (int64_t base = 0;; base += kAggUnroll * kThreads) {
#pragma unroll
    for (int u = 0; u < kAggUnroll; ++u) {
      const bool in = base + u * kThreads + threadIdx.x < tile;
      sums[0] += in ? agg[u].x : 0;
      sums[1] += in ? agg[u].y : 0;
      sums[2] += in ? agg[u].z : 0;
      sums[3] += in ? agg[u].w : 0;
    }
    if (base + kAggUnroll * kThreads >= tile) break;
#pragma unroll
    for (int u = 0; u < kAggUnroll; ++u) {
      const int64_t i = base + kAggUnroll * kThreads + u * kThreads + threadIdx.x;
      agg[u] = a.tile_agg[i < tile ? i : 0];
    }
  }
  // The tile's requests, from counts of offsets <= x over off[0, B]:
  //   owned  [own_lo, own_hi): start in [t0, t1), the last tile also at t1
  //   tokens [w0, tok_hi):     hold the tile's tokens (w0 = own_lo - 1)
  //   closed [close_lo - 1, close_hi - 1): end in (t0, t1], tile 0 also at 0
  const int64_t x[kWaves] = {t0 - 1, t1 - 1, t0, t1};
  tile_masks<STEPS, STAGED>(a, sh, t0, t1, x, kb, bps, fps);
  const TileMasks<T::kBlks>& m = sh.m;
  const Requests<STEPS, STAGED> rq{a, sh};
  const int64_t n_off = static_cast<int64_t>(a.n_requests) + 1;
  const int64_t own_lo = sh.s_count[0];
  const int64_t tok_hi = sh.s_count[1];
  const int64_t own_hi = last_tile ? n_off : tok_hi;
  const int64_t close_lo = tile == 0 ? 1 : sh.s_count[2];
  const int64_t close_hi = sh.s_count[3];
  const int64_t w0 = own_lo > 0 ? own_lo - 1 : 0;
  const int count = tok_hi - w0 <= kWindow ? static_cast<int>(tok_hi - w0) : -1;
  // request w0 starts in an earlier tile j0 and ends in this one
  const bool spans_in = own_lo > 0 && close_lo - 1 == w0 && close_lo < close_hi;

  __shared__ int64_t woff[kWindow + 1];
  __shared__ int64_t wgen[kWindow];
  __shared__ int32_t* wrow[kWindow];
  if (count >= 0)
    for (int k = threadIdx.x; k <= count; k += kThreads) {
      const int64_t b = w0 + k;
      woff[k] = rq.off(b);
      if (k < count) wrow[k] = rq.row(b);
    }
  __shared__ int64_t red[kWaves][kCounters];
  block_sums<kCounters>(sums, red);
  // sums: kept, moved, retired (and generated, not staged) before the tile

  // The start of request w0: the prefix at tile j0's end minus the tokens
  // of tile j0 from the request's first one, i.e. this tile's prefix minus
  // the aggregates of tiles (j0, tile) minus a recount of that stretch.
  __shared__ int64_t span_start[3];
  if (spans_in) {
    const int64_t lo = rq.off(w0);
    const int64_t j0 = lo / T::kTile;
    const int64_t hi = (j0 + 1) * T::kTile;  // < t0 <= total
    int64_t v[3] = {0, 0, 0};
    for (int64_t i = j0 + 1 + threadIdx.x; i < tile; i += kThreads) {
      const int4 g = a.tile_agg[i];
      v[0] += g.x;
      v[1] += g.y;
      v[2] += g.z;
    }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int64_t t = lo + s * kThreads + threadIdx.x;
      const bool valid = t < hi;
      const int64_t tc = valid ? t : lo;
      const uint8_t k = a.keep[tc];
      const int32_t bp = a.birth[tc], fp = a.final_pos[tc];
      const bool kept = valid && k != 0;
      const bool moved = kept && bp != fp;
      v[0] += kept;
      v[1] += moved;
      v[2] += valid && (!kept || moved);
    }
    __shared__ int64_t red3[kWaves][3];
    block_sums<3>(v, red3);
    if (threadIdx.x == 0)
#pragma unroll
      for (int c = 0; c < 3; ++c) span_start[c] = sums[c] - v[c];
  }

  // requests that start in the tile: kv_indptr, the generated tail of the
  // request before
  int64_t gen_total;
  if constexpr (STAGED) {
    gen_total = sh.s_genx[a.n_requests];
    for (int64_t b = own_lo + threadIdx.x; b < own_hi; b += kThreads) {
      const int64_t ob = rq.off(b);
      const int64_t at = sums[0] + m.count_before(ob - t0, 0) + sh.s_genx[b];  // kv_indptr[b]
      if (a.kv_indptr) a.kv_indptr[b] = static_cast<int32_t>(at);
      const int64_t g = b > 0 ? rq.gen(b - 1) : 0;
      if (g > 0 && a.kv_indices) {
        const int32_t* row = rq.row(b - 1);
        const int64_t n = ob - rq.off(b - 1);
        for (int64_t i = 0; i < g; ++i)
          if (at - g + i >= 0 && at - g + i < a.kv_capacity) a.kv_indices[at - g + i] = row[n + i];
      }
    }
  } else {
    int64_t carry = sums[3];
    for (int64_t base = own_lo; base < own_hi; base += kThreads) {
      const int64_t b = base + threadIdx.x;
      const bool mine = b < own_hi;
      int64_t pre, sum;
      block_scan(mine ? rq.gen(b) : 0, sh.lds, pre, sum);
      if (mine) {
        const int64_t gen_b = carry + pre;
        const int64_t ob = rq.off(b);
        const int64_t at = sums[0] + m.count_before(ob - t0, 0) + gen_b;  // kv_indptr[b]
        if (a.kv_indptr) a.kv_indptr[b] = static_cast<int32_t>(at);
        const int64_t g = b > 0 ? rq.gen(b - 1) : 0;
        if (g > 0 && a.kv_indices) {
          const int32_t* row = rq.row(b - 1);
          const int64_t n = ob - rq.off(b - 1);
          for (int64_t i = 0; i < g; ++i)
            if (at - g + i >= 0 && at - g + i < a.kv_capacity) a.kv_indices[at - g + i] = row[n + i];
        }
        if (count >= 0) {
          if (b - w0 < count) wgen[b - w0] = gen_b;
        } else {
          __hip_atomic_store(a.req_gen + b, gen_b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      carry += sum;
    }
    if (count >= 0 && own_lo > 0 && threadIdx.x == 0) wgen[0] = sums[3] - rq.gen(w0);
    gen_total = carry;  // the last tile's carry: every generated entry
  }
  if (last_tile && threadIdx.x == 0 && a.status) {
    const int64_t kept = sums[0] + m.before[T::kBlks][0];
    const int64_t moved = sums[1] + m.before[T::kBlks][1];
    const int64_t retired = sums[2] + m.before[T::kBlks][2];
    const bool bad = moved != a.fresh_count || kept > a.kept_capacity || retired > a.retired_capacity ||
                     (a.kv_indices && kept + gen_total > a.kv_capacity);
    a.status[0] = bad ? 1 : 0;
  }
  if (spans_in) __syncthreads();  // span_start

  // requests that end in the tile: counts and last-page lengths
  for (int64_t i = close_lo + threadIdx.x; i < close_hi; i += kThreads) {
    const int64_t b = i - 1;
    const int64_t lo = rq.off(b), hi = rq.off(i);
    int64_t start[3], end[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      end[c] = sums[c] + m.count_before(hi - t0, c);
      start[c] = lo >= t0 ? sums[c] + m.count_before(lo - t0, c) : span_start[c];  // lo < t0: b == w0
    }
    const int64_t kept = end[0] - start[0];
    if (a.counts) {
      a.counts[3 * b] = static_cast<int32_t>(kept);
      a.counts[3 * b + 1] = static_cast<int32_t>(end[1] - start[1]);
      a.counts[3 * b + 2] = static_cast<int32_t>(end[2] - start[2]);
    }
    if (a.last_page_len) {
      const int64_t len = kept + rq.gen(b);
      a.last_page_len[b] = len > 0 ? static_cast<int32_t>((len - 1) % a.page_size + 1) : 0;
    }
  }
  if (count < 0) {
    // the generated prefixes above are read back by other threads below
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));
  }
  __syncthreads();
  if (t1 <= t0) return;

  // Per-token outputs: every load first (birth slots, fresh slots), then
  // one wait, then the stores, so no store waits behind another.  Lanes
  // past t1 load for token t1 - 1 and store nothing.
  const int64_t fresh_last = a.fresh_count > 0 ? a.fresh_count - 1 : 0;
  if (count >= 0) {
    int32_t req[STEPS], slots[STEPS], fr[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int64_t t = t0 + s * kThreads + threadIdx.x;
      const int64_t tc = t < t1 ? t : t1 - 1;
      int l = 0, h = count - 1;  // woff[l] <= tc < woff[h + 1]
      while (l < h) {
        const int mid = (l + h + 1) >> 1;
        if (woff[mid] <= tc)
          l = mid;
        else
          h = mid - 1;
      }
      req[s] = l;
      // the birth slot: from the flat vector, else from the raw row
      const int32_t* sp = a.birth_slots ? a.birth_slots + tc : wrow[l] + (tc - woff[l]);
      slots[s] = *sp;
      const int p = s * kWaves + w;
      const int64_t pm = sums[1] + m.before[p][1] + rank_below(m.bits[p][1]);
      const int32_t f = a.fresh[pm < fresh_last ? pm : fresh_last];
      fr[s] = pm < a.fresh_count ? f : -1;
    }
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));  // vmcnt(0)
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int64_t t = t0 + s * kThreads + threadIdx.x;
      if (t >= t1) continue;
      const int p = s * kWaves + w;
      const int l = req[s];
      int64_t shift;
      if constexpr (STAGED)
        shift = sh.s_genx[w0 + l];
      else
        shift = wgen[l];
      emit_token(a, kb[s] != 0, bps[s], fps[s], slots[s], fr[s], sums[0] + m.before[p][0] + rank_below(m.bits[p][0]),
                 sums[1] + m.before[p][1] + rank_below(m.bits[p][1]),
                 sums[2] + m.before[p][2] + rank_below(m.bits[p][2]), wrow[l], t - woff[l], shift);
    }
  } else {
    // more requests than the window: look each token's request up
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int64_t t = t0 + s * kThreads + threadIdx.x;
      if (t >= t1) continue;
      int64_t l = w0, h = tok_hi - 1;
      while (l < h) {
        const int64_t mid = (l + h + 1) >> 1;
        if (rq.off(mid) <= t)
          l = mid;
        else
          h = mid - 1;
      }
      int32_t* row = rq.row(l);
      const int64_t local = t - rq.off(l);
      int64_t shift;
      if constexpr (STAGED)
        shift = sh.s_genx[l];
      else
        shift = l >= own_lo ? __hip_atomic_load(a.req_gen + l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : sums[3] - rq.gen(l);
      const int p = s * kWaves + w;
      const int64_t pm = sums[1] + m.before[p][1] + rank_below(m.bits[p][1]);
      const bool moved = kb[s] != 0 && bps[s] != fps[s];
      const int32_t slot = a.birth_slots ? a.birth_slots[t] : row[local];
      const int32_t fresh = (moved && pm < a.fresh_count) ? a.fresh[pm] : -1;
      emit_token(a, kb[s] != 0, bps[s], fps[s], slot, fresh, sums[0] + m.before[p][0] + rank_below(m.bits[p][0]), pm,
                 sums[2] + m.before[p][2] + rank_below(m.bits[p][2]), row, local, shift);
    }
  }
}

// Byte offsets of the workspace arrays (each 128-byte aligned).
struct Layout {
  int64_t tile_agg, req_gen, req_row, bytes;
};

Layout workspace_layout(int64_t n_requests, int64_t tiles) {
  Layout l{};
  int64_t at = 0;
  auto take = [&at](int64_t bytes) {
    const int64_t here = at;
    at += (bytes + 127) & ~static_cast<int64_t>(127);
    return here;
  };
  l.tile_agg = take(16 * tiles);
  l.req_gen = take(8 * (n_requests + 1));
  l.req_row = take(8 * n_requests);
  l.bytes = at;
  return l;
}

template <int STEPS, bool STAGED>
void launch(const CompactArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((count_kernel<STEPS, STAGED>), dim3(static_cast<unsigned>((a.tiles + kSuper - 1) / kSuper)),
                     dim3(kThreads), 0, st, a);
  hipLaunchKernelGGL((scatter_kernel<STEPS, STAGED>), dim3(static_cast<unsigned>(a.tiles)), dim3(kThreads), 0, st, a);
}

template <int STEPS>
void launch(const CompactArgs& a, hipStream_t st) {
  if (a.n_requests <= kStagedRequests)
    launch<STEPS, true>(a, st);
  else
    launch<STEPS, false>(a, st);
}

}  // namespace
}  // namespace akv

extern "C" int64_t akv_compact_workspace_bytes(int32_t n_requests, int64_t total_tokens) {
  using namespace akv;
  if (n_requests < 0 || total_tokens < 0) return -1;
  return workspace_layout(n_requests, tile_count(total_tokens, tile_steps(total_tokens))).bytes;
}

extern "C" int akv_compact_rows(int32_t n_requests, const int64_t* req_offsets, int64_t total_tokens,
                                int32_t* table, int64_t row_stride, const int64_t* row_pointers,
                                const int64_t* req_rows, const uint8_t* keep,
                                const int32_t* birth_positions, const int32_t* final_positions,
                                const int32_t* birth_slots, const int32_t* fresh_slots, int64_t fresh_count,
                                int32_t* retired, int64_t retired_capacity, int32_t* copy_src, int32_t* copy_dst,
                                int32_t* copy_pairs, int32_t* raw_indices, int32_t* active_positions,
                                int64_t kept_capacity, const int32_t* generated, int32_t* kv_indices,
                                int64_t kv_capacity, int32_t* kv_indptr, int32_t* last_page_len, int32_t page_size,
                                int32_t* counts, void* workspace, int64_t workspace_bytes, int32_t* status,
                                void* stream) {
  using namespace akv;
  if (n_requests < 0 || total_tokens < 0)
    return fail(AKV_EINVAL, "akv_compact_rows: negative request or token count");
  if (n_requests == 0) return AKV_OK;
  // lists may be null where their capacity is zero (every write is bounded by it)
  if (!req_offsets || !req_rows || !keep || !birth_positions || !final_positions || !workspace ||
      (retired_capacity > 0 && !retired) || (fresh_count > 0 && (!copy_src || !copy_dst || !copy_pairs)) ||
      (kept_capacity > 0 && (!raw_indices || !active_positions)))
    return fail(AKV_EINVAL, "akv_compact_rows: null device pointer");
  if (!row_pointers && !table)
    return fail(AKV_EINVAL, "akv_compact_rows: need a request table or row pointers");
  if (fresh_count > 0 && !fresh_slots)
    return fail(AKV_EINVAL, "akv_compact_rows: fresh_count > 0 with no fresh slots");
  if (last_page_len && page_size <= 0)
    return fail(AKV_EINVAL, "akv_compact_rows: page_size must be positive");
  if (generated && kv_indices && !kv_indptr)
    return fail(AKV_EINVAL, "akv_compact_rows: generated tokens need kv_indptr");
  const int steps = tile_steps(total_tokens);
  const int64_t tiles = tile_count(total_tokens, steps);
  if (tiles > 0x7fffffffLL)
    return fail(AKV_EINVAL, "akv_compact_rows: %lld tokens exceed one launch", static_cast<long long>(total_tokens));
  const Layout lay = workspace_layout(n_requests, tiles);
  if (workspace_bytes < lay.bytes)
    return fail(AKV_EINVAL, "akv_compact_rows: workspace holds %lld bytes, needs %lld",
                static_cast<long long>(workspace_bytes), static_cast<long long>(lay.bytes));
  if ((reinterpret_cast<uintptr_t>(workspace) & 15) != 0)
    return fail(AKV_EINVAL, "akv_compact_rows: workspace must be 16-byte aligned");

  CompactArgs a{};
  a.req_offsets = req_offsets;
  a.table = table;
  a.row_stride = row_stride;
  a.row_pointers = row_pointers;
  a.req_rows = req_rows;
  a.keep = keep;
  a.birth = birth_positions;
  a.final_pos = final_positions;
  a.birth_slots = birth_slots;
  a.fresh = fresh_count > 0 ? fresh_slots : static_cast<const int32_t*>(workspace);
  a.fresh_count = fresh_count;
  a.retired = retired;
  a.retired_capacity = retired_capacity;
  a.copy_src = copy_src;
  a.copy_dst = copy_dst;
  a.copy_pairs = copy_pairs;
  a.raw_indices = raw_indices;
  a.active_positions = active_positions;
  a.kept_capacity = kept_capacity;
  a.generated = generated;
  a.kv_indices = kv_indices;
  a.kv_capacity = kv_indices ? kv_capacity : 0;
  a.kv_indptr = kv_indptr;
  a.last_page_len = last_page_len;
  a.page_size = page_size > 0 ? page_size : 1;
  a.counts = counts;
  a.status = status;
  char* ws = static_cast<char*>(workspace);
  a.tile_agg = reinterpret_cast<int4*>(ws + lay.tile_agg);
  a.req_gen = reinterpret_cast<int64_t*>(ws + lay.req_gen);
  a.req_row = reinterpret_cast<int32_t**>(ws + lay.req_row);
  a.total = total_tokens;
  a.tiles = tiles;
  a.n_requests = n_requests;

  hipStream_t st = as_stream(stream);
  switch (steps) {
    case 1:
      launch<1>(a, st);
      break;
    case 2:
      launch<2>(a, st);
      break;
    default:
      launch<4>(a, st);
  }
  return check_launch("akv_compact_rows");
}
