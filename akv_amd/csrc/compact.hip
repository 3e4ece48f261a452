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
// Tiles of 256 x STEPS tokens of the concatenated batch, one of two paths:
//   one launch (fused_kernel; at most 512 requests, fewer than 2^29 tokens,
//            and a tile size whose tiles all fit on the device at once):
//            each tile loads its inputs once, publishes its counts, and
//            groups of 64 consecutive tiles are released in order by their
//            last arrival (see the one-launch section below);
//   two launches (count_kernel, scatter_kernel; every other batch, STEPS
//            growing until the batch is about 2048 tiles): per-tile
//            aggregates, then each tile sums every earlier tile's aggregate
//            (16 bytes each, read in one unrolled batch of up to 2304 issued
//            with the tile's own inputs) and writes every output it owns.
// Both write their outputs through tile_outputs.  A single-pass scan with a
// per-tile decoupled look-back measured slower on the ragged batch: per-tile
// chains of dependent global round trips (publish, poll, read) cost ~10 us
// under load, and 2048 tiles do not all fit on the chip at once.
//
// Loads are unconditional, from indices clamped into range, with the value
// selected afterwards: a load under a divergent condition is followed by a
// wait for every load in flight, which serialises the tile.  Batches of up
// to 512 requests keep their offsets, generated counts and rows in LDS
// (STAGED); larger ones read them from memory.
#include <atomic>

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
  uint64_t* tile_pack; // [tiles] one-launch path: tagged kept, moved of each tile
  int2* tile_pre;      // [tiles + 1] one-launch path: kept, moved before each tile
  uint64_t* req_local; // [B] one-launch path: tagged kept, moved of a request's first tile before it
  uint32_t* tile_fail; // [kFusedMaxTiles] one-launch path: tag of the call in which the tile withdrew
  uint32_t* sync;      // one-launch path: barrier words, zero before first use
  int32_t groups;      // one-launch path: arrival groups
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

// A wave-uniform 64-bit value moved to scalar registers.
__device__ __forceinline__ int64_t uniform(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint64_t>(v)));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
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

// Element i of a flat output through a 32-bit byte offset from the array
// base (i < 2^29), so the store takes a scalar base and one offset register.
__device__ __forceinline__ void put32(int32_t* base, uint32_t i, int32_t v) {
  *reinterpret_cast<int32_t*>(reinterpret_cast<char*>(base) + (i << 2)) = v;
}

// emit_token for batches whose positions and output sizes stay below 2^29.
__device__ __forceinline__ void emit_token32(const CompactArgs& a, bool kept, int32_t bpos, int32_t fpos,
                                             int32_t slot, int32_t fresh, uint32_t pk, uint32_t pm, uint32_t pr,
                                             int32_t* row, int32_t local, uint32_t shift) {
  const bool moved = kept && bpos != fpos;
  const bool retired = !kept || moved;
  int32_t terminal = -1;
  if (moved) {
    terminal = fresh;
    if (pm < a.fresh_count) {
      put32(a.copy_src, pm, slot);
      put32(a.copy_dst, pm, fresh);
      put32(a.copy_pairs, 2 * pm, bpos);
      put32(a.copy_pairs, 2 * pm + 1, fpos);
    }
  } else if (kept) {
    terminal = slot;
  }
  if (retired && pr < a.retired_capacity) put32(a.retired, pr, slot);
  if (kept && pk < a.kept_capacity) {
    put32(a.raw_indices, pk, local);
    put32(a.active_positions, pk, fpos);
  }
  if (kept && a.kv_indices && pk + shift < a.kv_capacity) put32(a.kv_indices, pk + shift, terminal);
  row[local] = terminal;
}

// The tile's requests, from counts of offsets <= x over off[0, B] (found by
// tile_masks):
//   owned  [own_lo, own_hi): start in [t0, t1), the last tile also at t1
//   tokens [w0, tok_hi):     hold the tile's tokens (w0 = own_lo - 1)
//   closed [close_lo - 1, close_hi - 1): end in (t0, t1], tile 0 also at 0
struct TileRequests {
  int64_t own_lo, own_hi, tok_hi, close_lo, close_hi, w0;
  int count;      // requests holding the tile's tokens, or -1 past kWindow
  bool spans_in;  // request w0 starts in an earlier tile and ends in this one
};

template <int STEPS, bool STAGED>
__device__ __forceinline__ TileRequests tile_requests(const CompactArgs& a, const Tile<STEPS, STAGED>& sh,
                                                      int64_t tile) {
  TileRequests r;
  r.own_lo = uniform(sh.s_count[0]);
  r.tok_hi = uniform(sh.s_count[1]);
  r.own_hi = tile == a.tiles - 1 ? static_cast<int64_t>(a.n_requests) + 1 : r.tok_hi;
  r.close_lo = tile == 0 ? 1 : uniform(sh.s_count[2]);
  r.close_hi = uniform(sh.s_count[3]);
  r.w0 = r.own_lo > 0 ? r.own_lo - 1 : 0;
  r.count = r.tok_hi - r.w0 <= kWindow ? static_cast<int>(r.tok_hi - r.w0) : -1;
  r.spans_in = r.own_lo > 0 && r.close_lo - 1 == r.w0 && r.close_lo < r.close_hi;
  return r;
}

// Offsets, generated prefixes and raw rows of the requests holding the
// tile's tokens, in LDS.
struct Window {
  int64_t off[kWindow + 1];
  int64_t gen[kWindow];
  int32_t* row[kWindow];
};

template <int STEPS, bool STAGED>
__device__ __forceinline__ void fill_window(const Requests<STEPS, STAGED>& rq, const TileRequests& r, Window& win) {
  if (r.count >= 0)
    for (int k = threadIdx.x; k <= r.count; k += kThreads) {
      const int64_t b = r.w0 + k;
      win.off[k] = rq.off(b);
      if (k < r.count) win.row[k] = rq.row(b);
    }
}

// Every output of the tile, from its exclusive prefix `sums` and, when
// spans_in, the start counts of request w0.  With status_bits >= 0 the last
// tile also writes the status word: its size check (bit 0) | status_bits.
// A token's kept flag comes from the tile's ballots, and its rank among retired tokens from the identity
// retired-before = tokens-before - kept-before + moved-before.  SMALL
// batches (positions and output sizes below 2^29) keep token positions and
// ranks in 32 bits.
template <int STEPS, bool STAGED, bool SMALL>
__device__ __forceinline__ void tile_outputs(const CompactArgs& a, Tile<STEPS, STAGED>& sh, Window& win,
                                             const TileRequests& r, int64_t tile, int64_t t0, int64_t t1,
                                             const int64_t (&sums)[kCounters], const int64_t (&span_start)[3],
                                             const int32_t (&bps)[STEPS], const int32_t (&fps)[STEPS],
                                             const int32_t (&slot0)[STEPS], int status_bits) {
  using T = Tile<STEPS, STAGED>;
  const int w = threadIdx.x >> 6;
  const TileMasks<T::kBlks>& m = sh.m;
  const Requests<STEPS, STAGED> rq{a, sh};
  // requests that start in the tile: kv_indptr, the generated tail of the
  // request before
  int64_t gen_total;
  if constexpr (STAGED) {
    gen_total = sh.s_genx[a.n_requests];
    for (int64_t b = r.own_lo + threadIdx.x; b < r.own_hi; b += kThreads) {
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
    for (int64_t base = r.own_lo; base < r.own_hi; base += kThreads) {
      const int64_t b = base + threadIdx.x;
      const bool mine = b < r.own_hi;
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
        if (r.count >= 0) {
          if (b - r.w0 < r.count) win.gen[b - r.w0] = gen_b;
        } else {
          __hip_atomic_store(a.req_gen + b, gen_b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      carry += sum;
    }
    if (r.count >= 0 && r.own_lo > 0 && threadIdx.x == 0) win.gen[0] = sums[3] - rq.gen(r.w0);
    gen_total = carry;  // the last tile's carry: every generated entry
  }
  if (status_bits >= 0 && tile == a.tiles - 1 && threadIdx.x == 0 && a.status) {
    const int64_t kept = sums[0] + m.before[T::kBlks][0];
    const int64_t moved = sums[1] + m.before[T::kBlks][1];
    const int64_t retired = sums[2] + m.before[T::kBlks][2];
    const bool bad = moved != a.fresh_count || kept > a.kept_capacity || retired > a.retired_capacity ||
                     (a.kv_indices && kept + gen_total > a.kv_capacity);
    a.status[0] = (bad ? 1 : 0) | status_bits;
  }

  // requests that end in the tile: counts and last-page lengths
  for (int64_t i = r.close_lo + threadIdx.x; i < r.close_hi; i += kThreads) {
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
  if (r.count < 0) {
    // the generated prefixes above are read back by other threads below
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));
  }
  __syncthreads();
  if (t1 <= t0) return;

  // Per-token outputs: every load first (birth slots from the raw rows,
  // fresh slots), then one wait, then the stores, so no store waits behind
  // another.  Lanes past t1 load for token t1 - 1 and store nothing.
  const int64_t fresh_last = a.fresh_count > 0 ? a.fresh_count - 1 : 0;
  if (SMALL && r.count >= 0) {
    const int32_t k0 = static_cast<int32_t>(sums[0]), m0 = static_cast<int32_t>(sums[1]);
    const int32_t u0 = static_cast<int32_t>(t0), u1 = static_cast<int32_t>(t1);
    const int32_t flast = static_cast<int32_t>(fresh_last);
    // the request holding token tc (a search of the window)
    auto find = [&](int32_t tc) {
      int l = 0, h = r.count - 1;  // off[l] <= tc < off[h + 1]
      while (l < h) {
        const int mid = (l + h + 1) >> 1;
        if (static_cast<int32_t>(win.off[mid]) <= tc)
          l = mid;
        else
          h = mid - 1;
      }
      return l;
    };
    int32_t slots[STEPS], fr[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int32_t t = u0 + s * kThreads + static_cast<int32_t>(threadIdx.x);
      const int32_t tc = t < u1 ? t : u1 - 1;
      if (a.birth_slots) {
        slots[s] = slot0[s];
      } else {
        const int l = find(tc);
        slots[s] = win.row[l][tc - static_cast<int32_t>(win.off[l])];
      }
      const int p = s * kWaves + w;
      const int32_t pm = m0 + m.before[p][1] + rank_below(m.bits[p][1]);
      const int32_t f = a.fresh[pm < flast ? pm : flast];
      fr[s] = pm < a.fresh_count ? f : -1;
    }
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));  // vmcnt(0)
    asm volatile("" ::: "memory");  // the searches below are redone, not kept in registers
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int32_t t = u0 + s * kThreads + static_cast<int32_t>(threadIdx.x);
      if (t >= u1) continue;
      const int p = s * kWaves + w;
      const int l = find(t);
      const uint64_t kbits = m.bits[p][0];
      const int32_t pk = k0 + m.before[p][0] + rank_below(kbits);
      const int32_t pm = m0 + m.before[p][1] + rank_below(m.bits[p][1]);
      emit_token32(a, (kbits >> lane_id()) & 1, bps[s], fps[s], slots[s], fr[s], pk, pm, t - pk + pm, win.row[l],
                   t - static_cast<int32_t>(win.off[l]), static_cast<uint32_t>(sh.s_genx[r.w0 + l]));
    }
  } else if (r.count >= 0) {
    int32_t req[STEPS], slots[STEPS], fr[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int64_t t = t0 + s * kThreads + threadIdx.x;
      const int64_t tc = t < t1 ? t : t1 - 1;
      int l = 0, h = r.count - 1;  // off[l] <= tc < off[h + 1]
      while (l < h) {
        const int mid = (l + h + 1) >> 1;
        if (win.off[mid] <= tc)
          l = mid;
        else
          h = mid - 1;
      }
      req[s] = l;
      // the birth slot: from the flat vector (already loaded), else the raw row
      slots[s] = a.birth_slots ? slot0[s] : win.row[l][tc - win.off[l]];
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
        shift = sh.s_genx[r.w0 + l];
      else
        shift = win.gen[l];
      const uint64_t kbits = m.bits[p][0];
      const int64_t pk = sums[0] + m.before[p][0] + rank_below(kbits);
      const int64_t pm = sums[1] + m.before[p][1] + rank_below(m.bits[p][1]);
      emit_token(a, (kbits >> lane_id()) & 1, bps[s], fps[s], slots[s], fr[s], pk, pm, t - pk + pm, win.row[l],
                 t - win.off[l], shift);
    }
  } else {
    // more requests than the window: look each token's request up
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int64_t t = t0 + s * kThreads + threadIdx.x;
      if (t >= t1) continue;
      int64_t l = r.w0, h = r.tok_hi - 1;
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
        shift = l >= r.own_lo ? __hip_atomic_load(a.req_gen + l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : sums[3] - rq.gen(l);
      const int p = s * kWaves + w;
      const uint64_t kbits = m.bits[p][0];
      const bool kept = (kbits >> lane_id()) & 1;
      const int64_t pk = sums[0] + m.before[p][0] + rank_below(kbits);
      const int64_t pm = sums[1] + m.before[p][1] + rank_below(m.bits[p][1]);
      const bool moved = kept && bps[s] != fps[s];
      const int32_t slot = a.birth_slots ? slot0[s] : row[local];
      const int32_t fresh = (moved && pm < a.fresh_count) ? a.fresh[pm] : -1;
      emit_token(a, kept, bps[s], fps[s], slot, fresh, pk, pm, t - pk + pm, row, local, shift);
    }
  }
}

// Birth slots from the flat vector, in the same round as the other inputs.
template <int STEPS>
__device__ __forceinline__ void load_birth_slots(const CompactArgs& a, int64_t t0, int64_t t1,
                                                 int32_t (&slot0)[STEPS]) {
#pragma unroll
  for (int s = 0; s < STEPS; ++s) slot0[s] = 0;
  if (!a.birth_slots || t1 <= t0) return;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int64_t t = t0 + s * kThreads + threadIdx.x;
    slot0[s] = a.birth_slots[t < t1 ? t : t1 - 1];
  }
}

// Two-launch path, second launch: per tile, the exclusive prefix summed from
// every earlier tile's aggregate, then every output the tile owns.
template <int STEPS, bool STAGED>
__global__ void __launch_bounds__(kThreads) scatter_kernel(const CompactArgs a) {
  using T = Tile<STEPS, STAGED>;
  __shared__ T sh;
  __shared__ Window win;
  const int64_t tile = blockIdx.x;
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
  int32_t bps[STEPS], fps[STEPS], slot0[STEPS];
  load_inputs<STEPS>(a, t0, t1, kb, bps, fps);
  load_birth_slots<STEPS>(a, t0, t1, slot0);
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
  const int64_t x[kWaves] = {t0 - 1, t1 - 1, t0, t1};
  tile_masks<STEPS, STAGED>(a, sh, t0, t1, x, kb, bps, fps);
  const TileRequests r = tile_requests<STEPS, STAGED>(a, sh, tile);
  const Requests<STEPS, STAGED> rq{a, sh};
  fill_window<STEPS, STAGED>(rq, r, win);
  __shared__ int64_t red[kWaves][kCounters];
  block_sums<kCounters>(sums, red);
  // sums: kept, moved, retired (and generated, not staged) before the tile

  // The start of request w0: the prefix at tile j0's end minus the tokens
  // of tile j0 from the request's first one, i.e. this tile's prefix minus
  // the aggregates of tiles (j0, tile) minus a recount of that stretch.
  __shared__ int64_t span_start[3];
  if (r.spans_in) {
    const int64_t lo = rq.off(r.w0);
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
    __syncthreads();
  }
  int64_t start_w0[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) start_w0[c] = r.spans_in ? span_start[c] : 0;
  tile_outputs<STEPS, STAGED, false>(a, sh, win, r, tile, t0, t1, sums, start_w0, bps, fps, slot0, 0);
}

// ---- One-launch path -------------------------------------------------------
//
// A tile loads its inputs once, publishes its kept and moved counts (and,
// for the requests that start in it, their counts before their first token;
// retired counts follow from tokens - kept + moved) and arrives at its
// group: 64 consecutive tiles.  The last tile to arrive in group k sums the
// group's counts, publishes the group's totals, reads the totals of groups
// 0 .. k-1 (one lane each), writes its tiles' exclusive prefixes (and, for
// the request holding the group's first token when it started in an earlier
// group, that request's start counts) and releases the group; each tile then
// writes its outputs.  Groups release in order as they fill, so the first
// tiles write while later ones still load.
//
// Every value one tile publishes for another carries the call's tag, epoch
// + 1 (finish_kernel advances the epoch once per call): tile counts, request
// start counts, group records and release words.  A reader therefore tells
// this call's values from earlier calls' and waits (bounded) until they are
// current; only the arrival counters are reset between calls (by each
// group's last arrival; the workspace is zero-filled before first use).
// Cross-tile values move by agent-scope atomic loads and stores, ordered by
// waiting for their completion: no cache-wide fence.
//
// Waits are bounded.  A tile whose wait runs out cancels its group's release
// word by compare-and-swap (a release and a withdrawal exclude each other),
// skips its outputs, records itself in the workspace and sets bit 2 of the
// status word.  finish_kernel, launched right after on the same stream,
// rebuilds the outputs of every withdrawn tile from the counts that every
// tile published, so the outputs are complete once the call's launches have
// run, whether or not all tiles could be resident at once (kernels of other
// streams holding CUs, a device smaller than the host assumed).  The host's
// residency check only picks the fast path; correctness does not rest on it.

constexpr int kGroupTiles = 64;  // tiles per group: one lane each
constexpr int kMaxGroups = 32;
constexpr int kSyncStride = 32;  // one 128-byte line per word
constexpr uint32_t kCancelled = 0x80000000u;
constexpr uint32_t kTagMask = 0x0fffffffu;
// polls of a bounded wait (one coherent load and a short sleep each: tens of
// milliseconds in all, orders of magnitude above any wait at this barrier
// when every tile is resident; a call whose tiles cannot all be resident
// stalls this long before its fallback)
constexpr uint32_t kPollLimit = 1u << 15;
constexpr int64_t kFusedMaxTiles = static_cast<int64_t>(kGroupTiles) * kMaxGroups;
// arrival counters, group records, release words, the epoch and the fail
// word (one line each), then the groups' span start counts
constexpr int kSpanWord = (3 * kMaxGroups + 2) * kSyncStride;
constexpr int64_t kSyncBytes = static_cast<int64_t>(kSpanWord + 2 * kMaxGroups) * 4;

// Data that one tile writes and another reads within the launch goes through
// agent-scope atomic loads and stores, which the device keeps coherent across
// its L2 slices without cache-wide write-back or invalidation; a writer waits
// for its stores to complete (vmcnt) before it signals.
__device__ __forceinline__ void put_pair(int2* p, int32_t x, int32_t y) {
  const uint64_t v = static_cast<uint64_t>(static_cast<uint32_t>(x)) | (static_cast<uint64_t>(static_cast<uint32_t>(y)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int2 get_pair(const int2* p) {
  const uint64_t v =
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_int2(static_cast<int32_t>(static_cast<uint32_t>(v)), static_cast<int32_t>(static_cast<uint32_t>(v >> 32)));
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8)); }
__device__ __forceinline__ uint64_t load64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t* arrive_word(const CompactArgs& a, int k) { return a.sync + k * kSyncStride; }
__device__ __forceinline__ uint64_t* record_word(const CompactArgs& a, int k) {
  return reinterpret_cast<uint64_t*>(a.sync + (kMaxGroups + k) * kSyncStride);
}
__device__ __forceinline__ uint32_t* release_word(const CompactArgs& a, int k) {
  return a.sync + (2 * kMaxGroups + k) * kSyncStride;
}
__device__ __forceinline__ uint32_t* epoch_word(const CompactArgs& a) { return a.sync + 3 * kMaxGroups * kSyncStride; }
__device__ __forceinline__ uint32_t* fail_word(const CompactArgs& a) {
  return a.sync + (3 * kMaxGroups + 1) * kSyncStride;
}
__device__ __forceinline__ int2* span_word(const CompactArgs& a, int k) {
  return reinterpret_cast<int2*>(a.sync + kSpanWord) + k;
}

// Tagged counts of a tile or of a request's first tile: tag in bits 32..63,
// moved in 16..31, kept in 0..15 (a tile holds at most 2048 tokens).
__device__ __forceinline__ uint64_t make_counts(uint32_t tag, int32_t kept, int32_t moved) {
  return (static_cast<uint64_t>(tag) << 32) | (static_cast<uint64_t>(static_cast<uint32_t>(moved)) << 16) |
         static_cast<uint32_t>(kept);
}
__device__ __forceinline__ uint32_t counts_tag(uint64_t v) { return static_cast<uint32_t>(v >> 32); }
__device__ __forceinline__ int32_t counts_kept(uint64_t v) { return static_cast<int32_t>(v & 0xffffu); }
__device__ __forceinline__ int32_t counts_moved(uint64_t v) { return static_cast<int32_t>((v >> 16) & 0xffffu); }

// A group record: tag in bits 36..63, kept tokens in 18..35, moved in 0..17
// (a group holds at most 64 x 2048 tokens).
__device__ __forceinline__ uint64_t make_record(uint32_t tag, uint32_t kept, uint32_t moved) {
  return (static_cast<uint64_t>(tag) << 36) | (static_cast<uint64_t>(kept) << 18) | moved;
}

// Thread 0 of a waiting tile: polls the group's release word.  True once
// released with `tag`; false when the group was cancelled or this tile
// withdrew (its wait ran out and it cancelled the group).
__device__ bool wait_release(uint32_t* word, uint32_t tag) {
  for (uint32_t polls = 0;; ++polls) {
    const uint32_t v = load32(word);
    if (v == tag) return true;
    if (v == (tag | kCancelled)) return false;
    if (polls >= kPollLimit) {
      uint32_t expected = v;
      if (__hip_atomic_compare_exchange_strong(word, &expected, tag | kCancelled, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        return false;
      return expected == tag;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Wave 0 of the last tile to arrive in group k: the group's totals, the
// totals of every earlier group, its tiles' prefixes, the start counts of
// the request that spans into the group, the release.  Returns
// (wave-uniform) whether the tiles' prefixes were written.
template <int STEPS>
__device__ bool release_group(const CompactArgs& a, const Tile<STEPS, true>& sh, int k, uint32_t tag) {
  using T = Tile<STEPS, true>;
  const int lane = lane_id();
  const int64_t first = static_cast<int64_t>(k) * kGroupTiles;
  const int count = static_cast<int>(a.tiles - first < kGroupTiles ? a.tiles - first : kGroupTiles);
  const int groups = a.groups;
  const int n = a.n_requests;
  // this group's tile counts, one per lane: every tile of the group has
  // arrived, so they are current unless the arrival counter was stale
  int32_t kt = 0, mt = 0;
  bool ok = true;
  {
    const int64_t i = first + (lane < count ? lane : 0);
    for (uint32_t polls = 0;; ++polls) {
      const uint64_t v = load64(a.tile_pack + i);
      const bool have = lane >= count || counts_tag(v) == tag;
      kt = lane < count ? counts_kept(v) : 0;
      mt = lane < count ? counts_moved(v) : 0;
      if (__ballot(!have) == 0) break;
      if (polls >= kPollLimit) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  const int32_t k_in = __ockl_wfscan_add_i32(kt, false);
  const int32_t m_in = __ockl_wfscan_add_i32(mt, false);
  const int32_t k_sum = __shfl(k_in + kt, 63);
  const int32_t m_sum = __shfl(m_in + mt, 63);
  if (lane == 0 && ok)
    __hip_atomic_store(record_word(a, k), make_record(tag, static_cast<uint32_t>(k_sum), static_cast<uint32_t>(m_sum)),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // The request holding the group's first token: when it started in an
  // earlier group g0 (tile j0), its start counts are g0's base + the counts
  // of g0's tiles before j0 + its own counts in tile j0, all published by
  // complete groups; read with the look-back.
  const int64_t t_first = first * T::kTile;
  int64_t w = wave_count_le(static_cast<int64_t>(n) + 1, t_first, [&](int64_t i) { return sh.s_off[i]; }) - 1;
  if (w > n - 1) w = n - 1;
  if (w < 0) w = 0;
  const int64_t lo = sh.s_off[w];
  const int64_t j0 = lo / T::kTile;
  const int g0 = static_cast<int>(j0 / kGroupTiles);
  const bool cross = lo < t_first && g0 < k;
  const bool in_start = cross && static_cast<int64_t>(g0) * kGroupTiles + lane < j0;
  // look back: the totals of groups 0 .. k-1 (one lane each), the start
  // group's tile counts before j0 (one lane each), the request's own counts
  int64_t bk = 0, bm = 0;
  int32_t sk = 0, sm = 0, lk = 0, lm = 0;
  if (ok) {
    const int ir = lane < k ? lane : 0;
    const int64_t is = cross ? static_cast<int64_t>(g0) * kGroupTiles + lane : 0;
    for (uint32_t polls = 0;; ++polls) {
      const uint64_t rec = load64(record_word(a, ir));
      const uint64_t vs = load64(a.tile_pack + is);
      const uint64_t vl = load64(a.req_local + w);
      const bool have = (lane >= k || static_cast<uint32_t>(rec >> 36) == tag) &&
                        (!in_start || counts_tag(vs) == tag) && (!cross || counts_tag(vl) == tag);
      bk = lane < k ? static_cast<int64_t>((rec >> 18) & 0x3ffffu) : 0;
      bm = lane < k ? static_cast<int64_t>(rec & 0x3ffffu) : 0;
      sk = in_start ? counts_kept(vs) : 0;
      sm = in_start ? counts_moved(vs) : 0;
      lk = counts_kept(vl);
      lm = counts_moved(vl);
      if (__ballot(!have) == 0) break;
      if (polls >= kPollLimit) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  const bool all_ok = __ballot(!ok) == 0;
  const int64_t base_k = __ockl_wfred_add_i64(bk);
  const int64_t base_m = __ockl_wfred_add_i64(bm);
  if (all_ok) {
    if (lane < count) put_pair(a.tile_pre + first + lane, static_cast<int32_t>(base_k + k_in), static_cast<int32_t>(base_m + m_in));
    if (k == groups - 1 && lane == 0)
      put_pair(a.tile_pre + a.tiles, static_cast<int32_t>(base_k + k_sum), static_cast<int32_t>(base_m + m_sum));
    if (cross) {
      const int64_t span_k = __ockl_wfred_add_i64((lane < g0 ? bk : 0) + sk) + lk;
      const int64_t span_m = __ockl_wfred_add_i64((lane < g0 ? bm : 0) + sm) + lm;
      if (lane == 0) put_pair(span_word(a, k), static_cast<int32_t>(span_k), static_cast<int32_t>(span_m));
    }
    wait_stores();
  }
  if (lane == 0) {
    // release (or cancel) the group; at most one withdrawal can change the
    // word first, after which the group stays cancelled
    uint32_t* word = release_word(a, k);
    const uint32_t want = all_ok ? tag : (tag | kCancelled);
    uint32_t cur = load32(word);
    for (int t = 0; t < 3 && cur != (tag | kCancelled); ++t) {
      uint32_t expected = cur;
      if (__hip_atomic_compare_exchange_strong(word, &expected, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        break;
      cur = expected;
    }
    if (k == groups - 1 && all_ok && a.status) {
      // every tile has arrived: the status word's final size check
      const int64_t kept = base_k + k_sum, moved = base_m + m_sum;
      const int64_t retired = a.total - kept + moved;
      const bool bad = moved != a.fresh_count || kept > a.kept_capacity || retired > a.retired_capacity ||
                       (a.kv_indices && kept + sh.s_genx[a.n_requests] > a.kv_capacity);
      uint32_t* st = reinterpret_cast<uint32_t*>(a.status);
      __hip_atomic_fetch_and(st, ~2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (bad) __hip_atomic_fetch_or(st, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  return all_ok;
}

// The batch's request offsets, rows and generated prefix in LDS (the
// one-launch path stages every request: at most kStagedRequests).
template <int STEPS>
__device__ __forceinline__ void stage_batch(const CompactArgs& a, Tile<STEPS, true>& sh) {
  constexpr int kRounds = (kStagedRequests + kThreads) / kThreads;  // B + 1 offsets
  const int n = a.n_requests;
  int64_t gv[kRounds];
#pragma unroll
  for (int q = 0; q < kRounds; ++q) {
    gv[q] = 0;
    if (q * kThreads > n) break;
    const int i = q * kThreads + threadIdx.x;
    const int ic = i < n ? i : n - 1;
    const int io = i <= n ? i : n;
    const int64_t o = a.req_offsets[io];
    const int64_t rr = a.req_rows[ic];
    const int32_t g = a.generated ? a.generated[ic] : 0;
    gv[q] = i < n ? g : 0;
    if (i <= n) sh.s_off[i] = o;
    if (i < n) sh.s_rr[i] = rr;
  }
  // exclusive prefix of generated entries over requests 0 .. B
  int64_t gcarry = 0;
#pragma unroll
  for (int q = 0; q < kRounds; ++q) {
    if (q * kThreads > n) break;
    int64_t pre, sum;
    block_scan(gv[q], sh.lds, pre, sum);
    const int i = q * kThreads + threadIdx.x;
    if (i <= n) sh.s_genx[i] = gcarry + pre;
    gcarry += sum;
  }
}

// Scalar registers are capped at 88 (86 reported): measured on MI355X, a
// 256-thread kernel holds 8 workgroups per CU up to 78 reported SGPRs, 7 up
// to 94 and 6 from 98, while the occupancy query reports 8 up to 94; the
// host applies the measured limit (kFusedMaxPerCu) when it picks the path.
template <int STEPS>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_num_sgpr(88))) fused_kernel(const CompactArgs a) {
  using T = Tile<STEPS, true>;
  __shared__ T sh;
  __shared__ Window win;
  __shared__ uint32_t s_sync[2];  // epoch, role
  __shared__ int32_t s_go[5];     // go, the tile's prefix (kept, moved), request w0's start (kept, moved)
  const int64_t tile = blockIdx.x;
  const int64_t t0 = tile * T::kTile;
  const int64_t t1 = t0 + T::kTile < a.total ? t0 + T::kTile : a.total;
  const int n = a.n_requests;
  const int k = static_cast<int>(tile / kGroupTiles);
  // the epoch goes to LDS only after the input loads are issued: stored at
  // once, its load would hold wave 0's inputs back by a round trip
  uint32_t epoch = 0;
  if (threadIdx.x == 0) {
    epoch = load32(epoch_word(a));
    // status bit 1 until the last group's look-back completes
    if (tile == 0 && a.status) __hip_atomic_store(a.status, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // one round of loads: the tile's inputs and flat birth slots, the batch's
  // request offsets, rows and generated counts
  uint8_t kb[STEPS];
  int32_t bps[STEPS], fps[STEPS], slot0[STEPS];
  load_inputs<STEPS>(a, t0, t1, kb, bps, fps);
  load_birth_slots<STEPS>(a, t0, t1, slot0);
  stage_batch<STEPS>(a, sh);
  if (threadIdx.x == 0) s_sync[0] = epoch;  // published by tile_masks' barriers
  const int64_t x[kWaves] = {t0 - 1, t1 - 1, t0, t1};
  tile_masks<STEPS, true>(a, sh, t0, t1, x, kb, bps, fps);
  const TileRequests r = tile_requests<STEPS, true>(a, sh, tile);
  const Requests<STEPS, true> rq{a, sh};
  fill_window<STEPS, true>(rq, r, win);
  // publish: the tile's counts, and the counts before each owned request
  // (s_sync[0] was written before the barriers of tile_masks' scans)
  const uint32_t tag = (s_sync[0] + 1u) & kTagMask;
  const TileMasks<T::kBlks>& m = sh.m;
  for (int64_t b = r.own_lo + threadIdx.x; b < r.own_hi && b < n; b += kThreads) {
    const int64_t q = rq.off(b) - t0;
    __hip_atomic_store(a.req_local + b, make_counts(tag, m.count_before(q, 0), m.count_before(q, 1)),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(a.tile_pack + tile, make_counts(tag, m.before[T::kBlks][0], m.before[T::kBlks][1]),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t gfirst = static_cast<int64_t>(k) * kGroupTiles;
    const uint32_t gsize = static_cast<uint32_t>(a.tiles - gfirst < kGroupTiles ? a.tiles - gfirst : kGroupTiles);
    uint32_t last = 0;
    if (__hip_atomic_fetch_add(arrive_word(a, k), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gsize - 1) {
      store32(arrive_word(a, k), 0u);
      last = 1;
    }
    s_sync[1] = last;
  }
  __syncthreads();
  if (s_sync[1]) {
    if (threadIdx.x < 64) {
      const bool ok = release_group<STEPS>(a, sh, k, tag);
      if (threadIdx.x == 0) s_go[0] = ok ? 1 : 0;
    }
  } else if (threadIdx.x == 0) {
    s_go[0] = wait_release(release_word(a, k), tag) ? 1 : 0;
  }
  if (threadIdx.x == 0) {
    bool go = s_go[0] != 0;
    if (go) {
      // the tile's prefix and, when a request spans in, its start counts:
      // from the group's span word when it started in an earlier group, else
      // from its first tile's prefix and its tagged counts there
      // (all loads issued before any LDS store consumes one: one round trip)
      const int2 pre = get_pair(a.tile_pre + tile);
      const int64_t j0 = r.spans_in ? rq.off(r.w0) / T::kTile : 0;
      const bool from_span = j0 < static_cast<int64_t>(k) * kGroupTiles;
      int2 start = make_int2(0, 0);
      uint64_t v = 0;
      if (r.spans_in) {
        if (from_span) {
          start = get_pair(span_word(a, k));
        } else {
          start = get_pair(a.tile_pre + j0);
          v = load64(a.req_local + r.w0);
        }
      }
      if (r.spans_in && !from_span) {
        for (uint32_t polls = 0; counts_tag(v) != tag && polls < kPollLimit; ++polls) {
          __builtin_amdgcn_s_sleep(2);
          v = load64(a.req_local + r.w0);
        }
        go = counts_tag(v) == tag;
        start.x += counts_kept(v);
        start.y += counts_moved(v);
      }
      s_go[1] = pre.x;
      s_go[2] = pre.y;
      s_go[3] = start.x;
      s_go[4] = start.y;
    }
    if (!go) {
      // withdraw: finish_kernel rebuilds this tile's outputs
      store32(a.tile_fail + tile, tag);
      store32(fail_word(a), tag);
      if (a.status) __hip_atomic_fetch_or(reinterpret_cast<uint32_t*>(a.status), 4u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    }
    s_go[0] = go ? 1 : 0;
  }
  __syncthreads();
  if (!s_go[0]) return;
  int64_t sums[kCounters];
  sums[0] = s_go[1];
  sums[1] = s_go[2];
  sums[2] = t0 - sums[0] + sums[1];
  sums[3] = 0;
  int64_t start_w0[3] = {0, 0, 0};
  if (r.spans_in) {
    start_w0[0] = s_go[3];
    start_w0[1] = s_go[4];
    start_w0[2] = rq.off(r.w0) - start_w0[0] + start_w0[1];
  }
  tile_outputs<STEPS, true, true>(a, sh, win, r, tile, t0, t1, sums, start_w0, bps, fps, slot0, -1);
}

// Right after the one-launch kernel, one workgroup: advances the epoch and,
// when tiles of the call withdrew, rebuilds their outputs -- every tile's
// prefix from the counts all tiles published, then each withdrawn tile's
// work as in the one-launch kernel, in order.  This is the fallback, not the
// fast path; it also resets the arrival counters and writes the final
// status (bit 2 kept: the outputs were rebuilt).
template <int STEPS>
__global__ void __launch_bounds__(kThreads) finish_kernel(const CompactArgs a) {
  using T = Tile<STEPS, true>;
  __shared__ T sh;
  __shared__ Window win;
  __shared__ uint32_t s_word[2];
  if (threadIdx.x == 0) {
    s_word[0] = load32(epoch_word(a));
    s_word[1] = load32(fail_word(a));
  }
  __syncthreads();
  const uint32_t epoch = s_word[0];
  const uint32_t tag = (epoch + 1u) & kTagMask;
  if (s_word[1] != tag) {
    if (threadIdx.x == 0) store32(epoch_word(a), epoch + 1u);
    return;
  }
  // every tile's exclusive prefix
  int64_t ck = 0, cm = 0;
  for (int64_t base = 0; base < a.tiles; base += kThreads) {
    const int64_t i = base + threadIdx.x;
    const uint64_t v = load64(a.tile_pack + (i < a.tiles ? i : 0));
    const int64_t kt = i < a.tiles ? counts_kept(v) : 0;
    const int64_t mt = i < a.tiles ? counts_moved(v) : 0;
    int64_t pk, sk, pm, sm;
    block_scan(kt, sh.lds, pk, sk);
    block_scan(mt, sh.lds, pm, sm);
    if (i < a.tiles) put_pair(a.tile_pre + i, static_cast<int32_t>(ck + pk), static_cast<int32_t>(cm + pm));
    ck += sk;
    cm += sm;
  }
  if (threadIdx.x == 0) put_pair(a.tile_pre + a.tiles, static_cast<int32_t>(ck), static_cast<int32_t>(cm));
  wait_stores();
  stage_batch<STEPS>(a, sh);
  __syncthreads();
  const Requests<STEPS, true> rq{a, sh};
  __shared__ uint8_t s_flag[kThreads];
  for (int64_t base = 0; base < a.tiles; base += kThreads) {
    // the tiles of this chunk that withdrew in this call
    const int64_t i = base + threadIdx.x;
    s_flag[threadIdx.x] = i < a.tiles && load32(a.tile_fail + i) == tag;
    __syncthreads();
    for (int u = 0; u < kThreads && base + u < a.tiles; ++u) {
      if (!s_flag[u]) continue;
      const int64_t tile = base + u;
      const int64_t t0 = tile * T::kTile;
      const int64_t t1 = t0 + T::kTile < a.total ? t0 + T::kTile : a.total;
      uint8_t kb[STEPS];
      int32_t bps[STEPS], fps[STEPS], slot0[STEPS];
      load_inputs<STEPS>(a, t0, t1, kb, bps, fps);
      load_birth_slots<STEPS>(a, t0, t1, slot0);
      const int64_t x[kWaves] = {t0 - 1, t1 - 1, t0, t1};
      tile_masks<STEPS, true>(a, sh, t0, t1, x, kb, bps, fps);
      const TileRequests r = tile_requests<STEPS, true>(a, sh, tile);
      fill_window<STEPS, true>(rq, r, win);
      const int2 pre = get_pair(a.tile_pre + tile);
      int64_t sums[kCounters];
      sums[0] = __builtin_amdgcn_readfirstlane(pre.x);
      sums[1] = __builtin_amdgcn_readfirstlane(pre.y);
      sums[2] = t0 - sums[0] + sums[1];
      sums[3] = 0;
      int64_t start_w0[3] = {0, 0, 0};
      if (r.spans_in) {
        const int64_t lo = rq.off(r.w0);
        const int2 pj = get_pair(a.tile_pre + lo / T::kTile);
        const uint64_t v = load64(a.req_local + r.w0);
        start_w0[0] = __builtin_amdgcn_readfirstlane(pj.x + counts_kept(v));
        start_w0[1] = __builtin_amdgcn_readfirstlane(pj.y + counts_moved(v));
        start_w0[2] = lo - start_w0[0] + start_w0[1];
      }
      tile_outputs<STEPS, true, true>(a, sh, win, r, tile, t0, t1, sums, start_w0, bps, fps, slot0, -1);
    }
    __syncthreads();
    if (i < a.tiles && s_flag[threadIdx.x]) store32(a.tile_fail + i, 0u);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (a.status) {
      const int64_t retired = a.total - ck + cm;
      const bool bad = cm != a.fresh_count || ck > a.kept_capacity || retired > a.retired_capacity ||
                       (a.kv_indices && ck + sh.s_genx[a.n_requests] > a.kv_capacity);
      store32(reinterpret_cast<uint32_t*>(a.status), (bad ? 1u : 0u) | 4u);
    }
    for (int g = 0; g < kMaxGroups; ++g) store32(arrive_word(a, g), 0u);
    store32(epoch_word(a), epoch + 1u);
  }
}

// Byte offsets of the workspace arrays (each 128-byte aligned).
struct Layout {
  int64_t sync, tile_fail, tile_agg, tile_prefix, req_local, req_gen, req_row, bytes;
};

// Sized for both paths: the barrier words and the withdrawn-tile words
// first (at fixed offsets, so batches of any size may share a workspace),
// then per-tile and per-request arrays.
Layout workspace_layout(int64_t n_requests, int64_t total) {
  const int64_t two_launch = tile_count(total, tile_steps(total));
  const int64_t per_step = (total + kThreads - 1) / kThreads;  // most tiles of the one-launch path
  const int64_t one_launch = per_step < kFusedMaxTiles ? per_step : kFusedMaxTiles;
  const int64_t tiles = two_launch > one_launch ? two_launch : one_launch;
  Layout l{};
  int64_t at = 0;
  auto take = [&at](int64_t bytes) {
    const int64_t here = at;
    at += (bytes + 127) & ~static_cast<int64_t>(127);
    return here;
  };
  l.sync = take(kSyncBytes);
  l.tile_fail = take(4 * kFusedMaxTiles);
  l.tile_agg = take(16 * tiles);
  l.tile_prefix = take(8 * (tiles + 1));
  l.req_local = take(8 * n_requests);
  l.req_gen = take(8 * (n_requests + 1));
  l.req_row = take(8 * n_requests);
  l.bytes = at;
  return l;
}

// One-launch tile sizes, in the order tried (the smallest that fits).
constexpr int kFusedSteps[] = {1, 2, 3, 4, 5, 6, 8};
constexpr int kFusedVariants = sizeof(kFusedSteps) / sizeof(kFusedSteps[0]);
constexpr int kMaxDevices = 64;
constexpr int kFusedMaxPerCu = 7;  // residency of fused_kernel's SGPR footprint (see its declaration)

const void* fused_entry(int steps) {
  switch (steps) {
    case 1: return reinterpret_cast<const void*>(&fused_kernel<1>);
    case 2: return reinterpret_cast<const void*>(&fused_kernel<2>);
    case 3: return reinterpret_cast<const void*>(&fused_kernel<3>);
    case 4: return reinterpret_cast<const void*>(&fused_kernel<4>);
    case 5: return reinterpret_cast<const void*>(&fused_kernel<5>);
    case 6: return reinterpret_cast<const void*>(&fused_kernel<6>);
    default: return reinterpret_cast<const void*>(&fused_kernel<8>);
  }
}

// Workgroups of fused_kernel<kFusedSteps[v]> resident at once on the current
// device (0 when unknown), cached per device: the occupancy query (registers,
// LDS) bounded by the measured SGPR limit.
int64_t fused_capacity(int v) {
  static std::atomic<int64_t> cache[kMaxDevices][kFusedVariants];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int64_t c = cache[dev][v].load(std::memory_order_relaxed);
  if (c > 0) return c;
  int blocks = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fused_entry(kFusedSteps[v]), kThreads, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  c = static_cast<int64_t>(blocks < kFusedMaxPerCu ? blocks : kFusedMaxPerCu) * cus;
  cache[dev][v].store(c, std::memory_order_relaxed);
  return c;
}

// The one-launch variant for a batch (index into kFusedSteps), or -1 when
// it takes the two-launch path: more than kStagedRequests requests, a size
// at or past 2^29 (32-bit byte offsets), or no tile size whose tiles all fit
// on the current device.
int fused_variant(int32_t n_requests, int64_t total_tokens, int64_t largest_list) {
  constexpr int64_t kSmall = int64_t{1} << 29;
  if (n_requests > kStagedRequests || total_tokens >= kSmall || largest_list >= kSmall) return -1;
  for (int v = 0; v < kFusedVariants; ++v) {
    const int64_t t = tile_count(total_tokens, kFusedSteps[v]);
    if (t <= kFusedMaxTiles && t <= fused_capacity(v)) return v;
  }
  return -1;
}

// The one-launch kernel, then the one-workgroup finish (epoch, fallback).
template <int STEPS>
void launch_fused(const CompactArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((fused_kernel<STEPS>), dim3(static_cast<unsigned>(a.tiles)), dim3(kThreads), 0, st, a);
  hipLaunchKernelGGL((finish_kernel<STEPS>), dim3(1), dim3(kThreads), 0, st, a);
}

void launch_fused(int steps, const CompactArgs& a, hipStream_t st) {
  switch (steps) {
    case 1: launch_fused<1>(a, st); break;
    case 2: launch_fused<2>(a, st); break;
    case 3: launch_fused<3>(a, st); break;
    case 4: launch_fused<4>(a, st); break;
    case 5: launch_fused<5>(a, st); break;
    case 6: launch_fused<6>(a, st); break;
    default: launch_fused<8>(a, st); break;
  }
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
  return workspace_layout(n_requests, total_tokens).bytes;
}

extern "C" int akv_compact_launches(int32_t n_requests, int64_t total_tokens, int64_t largest_list,
                                    int64_t* tile_tokens) {
  using namespace akv;
  if (n_requests < 0 || total_tokens < 0 || largest_list < 0) return fail(AKV_EINVAL, "akv_compact_launches: negative size");
  if (tile_tokens) *tile_tokens = 0;
  if (n_requests == 0) return 0;
  const int v = fused_variant(n_requests, total_tokens, largest_list);
  if (tile_tokens) *tile_tokens = static_cast<int64_t>(kThreads) * (v >= 0 ? kFusedSteps[v] : tile_steps(total_tokens));
  return v >= 0 ? 1 : 2;
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
  const Layout lay = workspace_layout(n_requests, total_tokens);
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
  a.sync = reinterpret_cast<uint32_t*>(ws + lay.sync);
  a.tile_agg = reinterpret_cast<int4*>(ws + lay.tile_agg);
  a.tile_pack = reinterpret_cast<uint64_t*>(ws + lay.tile_agg);  // the paths never share a call
  a.tile_fail = reinterpret_cast<uint32_t*>(ws + lay.tile_fail);
  a.tile_pre = reinterpret_cast<int2*>(ws + lay.tile_prefix);
  a.req_local = reinterpret_cast<uint64_t*>(ws + lay.req_local);
  a.req_gen = reinterpret_cast<int64_t*>(ws + lay.req_gen);
  a.req_row = reinterpret_cast<int32_t**>(ws + lay.req_row);
  a.total = total_tokens;
  a.tiles = tiles;
  a.n_requests = n_requests;

  hipStream_t st = as_stream(stream);
  int64_t largest = fresh_count > retired_capacity ? fresh_count : retired_capacity;
  if (kept_capacity > largest) largest = kept_capacity;
  if (kv_indices && kv_capacity > largest) largest = kv_capacity;
  const int v = fused_variant(n_requests, total_tokens, largest);
  if (v >= 0) {
    a.tiles = tile_count(total_tokens, kFusedSteps[v]);
    a.groups = static_cast<int32_t>((a.tiles + kGroupTiles - 1) / kGroupTiles);
    launch_fused(kFusedSteps[v], a, st);
    return check_launch("akv_compact_rows");
  }
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
