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
// Two or three launches, no inter-workgroup waiting:
//   1. count:   tiles of 256 x steps tokens per request (steps grows with the
//               batch so a single request still spreads over many
//               workgroups); wave ballots + popcount,
//               wave totals through LDS -> per-tile (kept, moved)
//   2. offsets: (batches of more than kFusedMaxEntries tiles only) one
//               workgroup scans the tile counts in request-major order ->
//               flat output offsets per tile, per-request counts, kv_indptr;
//               smaller batches derive these inside the scatter workgroups
//               from a block reduction over the earlier tiles' counts
//   3. scatter: same tiles again; ballot/mbcnt ranks inside each 256-token
//               step, LDS wave totals, running carry -> every output.
#include "common.h"

namespace akv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSteps = 16;  // at most 4096 tokens per workgroup
// Up to this many tiles per batch, each scatter workgroup derives its own
// offsets from the tile counts (2 launches); beyond, a scan launch does.
constexpr int64_t kFusedMaxEntries = 4096;

// Steps of 256 tokens per tile: about 1024 tiles over the whole batch.
int tile_steps(int32_t n_requests, int64_t max_tokens) {
  const int64_t work = static_cast<int64_t>(n_requests) * max_tokens;
  int steps = 1;
  while (steps < kMaxSteps && work > static_cast<int64_t>(kThreads) * steps * 1024) steps <<= 1;
  return steps;
}

int64_t tiles_per_request(int32_t n_requests, int64_t max_tokens) {
  const int64_t tile = static_cast<int64_t>(kThreads) * tile_steps(n_requests, max_tokens);
  return max_tokens <= 0 ? 1 : (max_tokens + tile - 1) / tile;
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
  const int32_t* fresh;
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
  // workspace
  int32_t* tile_counts;    // [B * tiles_per_req * 2] kept, moved
  int64_t* tile_offsets;   // [B * tiles_per_req * 3] kept, moved, retired (flat)
  int64_t* req_kv_base;    // [B] kv_indptr[b] as int64
  int64_t* req_kept;       // [B] kept tokens per request
  int32_t n_requests;
  int32_t tiles_per_req;
  int32_t steps;  // 256-token steps per tile
};

__device__ __forceinline__ int32_t* request_row(const CompactArgs& a, int b) {
  const int64_t r = a.req_rows[b];
  if (a.row_pointers) return reinterpret_cast<int32_t*>(a.row_pointers[r]);
  return a.table + r * a.row_stride;
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// number of set lanes below this one in a 64-bit ballot
__device__ __forceinline__ int rank_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

__global__ void __launch_bounds__(kThreads) compact_count_kernel(const CompactArgs a) {
  const int b = blockIdx.y;
  const int tile = blockIdx.x;
  const int64_t base = a.req_offsets[b];
  const int64_t n = a.req_offsets[b + 1] - base;
  const int64_t start = static_cast<int64_t>(tile) * kThreads * a.steps;
  __shared__ int wave_sums[2][kWaves];
  int kept = 0, moved = 0;
  if (start < n) {
    for (int s = 0; s < a.steps; ++s) {
      const int64_t i = start + s * kThreads + threadIdx.x;
      if (i < n) {
        const bool k = a.keep[base + i] != 0;
        kept += k;
        moved += k && (a.birth[base + i] != a.final_pos[base + i]);
      }
    }
  }
  // wave reduction, then the 4 wave totals through LDS
  for (int off = 32; off > 0; off >>= 1) {
    kept += __shfl_xor(kept, off);
    moved += __shfl_xor(moved, off);
  }
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0) {
    wave_sums[0][w] = kept;
    wave_sums[1][w] = moved;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int tk = 0, tm = 0;
    for (int q = 0; q < kWaves; ++q) {
      tk += wave_sums[0][q];
      tm += wave_sums[1][q];
    }
    const int64_t slot = (static_cast<int64_t>(b) * a.tiles_per_req + tile) * 2;
    a.tile_counts[slot] = tk;
    a.tile_counts[slot + 1] = tm;
  }
}

// One workgroup: exclusive scan of the tile counts in request-major order.
__global__ void __launch_bounds__(1024) compact_offsets_kernel(const CompactArgs a) {
  __shared__ int64_t carry[3];
  __shared__ int64_t wave_tot[16][3];
  const int64_t entries = static_cast<int64_t>(a.n_requests) * a.tiles_per_req;
  if (threadIdx.x < 3) carry[threadIdx.x] = 0;
  __syncthreads();
  for (int64_t base = 0; base < entries; base += blockDim.x) {
    const int64_t e = base + threadIdx.x;
    int64_t v[3] = {0, 0, 0};
    if (e < entries) {
      const int b = static_cast<int>(e / a.tiles_per_req);
      const int t = static_cast<int>(e - static_cast<int64_t>(b) * a.tiles_per_req);
      const int64_t n = a.req_offsets[b + 1] - a.req_offsets[b];
      const int64_t tile = static_cast<int64_t>(kThreads) * a.steps;
      const int64_t len = n - static_cast<int64_t>(t) * tile;
      const int64_t tile_len = len <= 0 ? 0 : (len < tile ? len : tile);
      v[0] = a.tile_counts[2 * e];
      v[1] = a.tile_counts[2 * e + 1];
      v[2] = tile_len - v[0] + v[1];
    }
    // inclusive wave scan
    int64_t inc[3] = {v[0], v[1], v[2]};
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        const int64_t up = __shfl_up(inc[c], off);
        if (lane_id() >= off) inc[c] += up;
      }
    }
    const int w = threadIdx.x >> 6;
    if (lane_id() == 63) {
#pragma unroll
      for (int c = 0; c < 3; ++c) wave_tot[w][c] = inc[c];
    }
    __syncthreads();
    int64_t prefix[3] = {carry[0], carry[1], carry[2]};
    for (int q = 0; q < w; ++q) {
#pragma unroll
      for (int c = 0; c < 3; ++c) prefix[c] += wave_tot[q][c];
    }
    if (e < entries) {
#pragma unroll
      for (int c = 0; c < 3; ++c) a.tile_offsets[3 * e + c] = prefix[c] + inc[c] - v[c];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      const int waves = (blockDim.x + 63) / 64;
      for (int q = 0; q < waves; ++q) {
#pragma unroll
        for (int c = 0; c < 3; ++c) carry[c] += wave_tot[q][c];
      }
    }
    __syncthreads();
  }
  // Per-request counts and kv_indptr (request totals from the tile offsets).
  __shared__ int64_t kv_carry;
  if (threadIdx.x == 0) kv_carry = 0;
  __syncthreads();
  for (int base = 0; base < a.n_requests; base += blockDim.x) {
    const int b = base + threadIdx.x;
    int64_t kept = 0, moved = 0, retired = 0, len = 0;
    if (b < a.n_requests) {
      const int64_t first = static_cast<int64_t>(b) * a.tiles_per_req;
      const int64_t next = first + a.tiles_per_req;
      const bool last = b + 1 == a.n_requests;
      const int64_t* o = a.tile_offsets;
      kept = (last ? carry[0] : o[3 * next]) - o[3 * first];
      moved = (last ? carry[1] : o[3 * next + 1]) - o[3 * first + 1];
      retired = (last ? carry[2] : o[3 * next + 2]) - o[3 * first + 2];
      len = kept + (a.generated ? a.generated[b] : 0);
      if (a.counts) {
        a.counts[3 * b] = static_cast<int32_t>(kept);
        a.counts[3 * b + 1] = static_cast<int32_t>(moved);
        a.counts[3 * b + 2] = static_cast<int32_t>(retired);
      }
    }
    int64_t inc = len;
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t up = __shfl_up(inc, off);
      if (lane_id() >= off) inc += up;
    }
    const int w = threadIdx.x >> 6;
    if (lane_id() == 63) wave_tot[w][0] = inc;
    __syncthreads();
    int64_t prefix = kv_carry;
    for (int q = 0; q < w; ++q) prefix += wave_tot[q][0];
    if (b < a.n_requests) {
      const int64_t excl = prefix + inc - len;
      a.req_kv_base[b] = excl;
      a.req_kept[b] = kept;
      if (a.kv_indptr) {
        if (b == 0) a.kv_indptr[0] = 0;
        a.kv_indptr[b + 1] = static_cast<int32_t>(excl + len);
      }
      if (a.last_page_len) a.last_page_len[b] = len > 0 ? static_cast<int32_t>((len - 1) % a.page_size + 1) : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      const int waves = (blockDim.x + 63) / 64;
      for (int q = 0; q < waves; ++q) kv_carry += wave_tot[q][0];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && a.status) {
    const bool bad = carry[1] != a.fresh_count || carry[0] > a.kept_capacity ||
                     carry[2] > a.retired_capacity || (a.kv_indices && kv_carry > a.kv_capacity);
    a.status[0] = bad ? 1 : 0;
  }
}

// Block-wide sum of K int64 accumulators (every thread gets the totals).
template <int K>
__device__ __forceinline__ void block_sum(int64_t (&v)[K], int64_t (*lds)[K]) {
#pragma unroll
  for (int k = 0; k < K; ++k)
    for (int off = 32; off > 0; off >>= 1) v[k] += __shfl_xor(v[k], off);
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) lds[w][k] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    v[k] = 0;
    for (int q = 0; q < kWaves; ++q) v[k] += lds[q][k];
  }
  __syncthreads();
}

// Tokens of tile entry e (request-major) for the tile size of this launch.
__device__ __forceinline__ int64_t tile_length(const CompactArgs& a, int64_t e) {
  const int rb = static_cast<int>(e / a.tiles_per_req);
  const int rt = static_cast<int>(e - static_cast<int64_t>(rb) * a.tiles_per_req);
  const int64_t tile = static_cast<int64_t>(kThreads) * a.steps;
  const int64_t len = a.req_offsets[rb + 1] - a.req_offsets[rb] - rt * tile;
  return len <= 0 ? 0 : (len < tile ? len : tile);
}

// FUSED: the tile's exclusive offsets, its request's kv base and the
// per-request outputs come from a block reduction over the tile counts of
// the earlier tiles (small batches: saves the offsets launch).  Otherwise
// they come from compact_offsets_kernel.
template <bool FUSED>
__global__ void __launch_bounds__(kThreads) compact_scatter_kernel(const CompactArgs a) {
  const int b = blockIdx.y;
  const int tile = blockIdx.x;
  const int64_t base = a.req_offsets[b];
  const int64_t n = a.req_offsets[b + 1] - base;
  const int64_t start = static_cast<int64_t>(tile) * kThreads * a.steps;
  int32_t* row = request_row(a, b);
  int64_t kv_base, req_kept_base, req_kept, carry_kept, carry_moved, carry_retired;
  if (FUSED) {
    __shared__ int64_t lds[kWaves][7];
    const int64_t first = static_cast<int64_t>(b) * a.tiles_per_req;
    const int64_t me = first + tile;
    const int64_t end = first + a.tiles_per_req;
    // 0-2: kept/moved/retired before this tile; 3: kept before the request;
    // 4-6: kept/moved/retired of the request
    int64_t v[7] = {0, 0, 0, 0, 0, 0, 0};
    for (int64_t e = threadIdx.x; e < end; e += kThreads) {
      const int64_t k = a.tile_counts[2 * e];
      const int64_t m = a.tile_counts[2 * e + 1];
      const int64_t r = tile_length(a, e) - k + m;
      if (e < me) {
        v[0] += k;
        v[1] += m;
        v[2] += r;
      }
      if (e < first) {
        v[3] += k;
      } else {
        v[4] += k;
        v[5] += m;
        v[6] += r;
      }
    }
    int64_t gen_before = 0;
    if (a.generated)
      for (int q = threadIdx.x; q < b; q += kThreads) gen_before += a.generated[q];
    int64_t g[1] = {gen_before};
    block_sum<7>(v, lds);
    block_sum<1>(g, reinterpret_cast<int64_t(*)[1]>(&lds[0][0]));
    carry_kept = v[0];
    carry_moved = v[1];
    carry_retired = v[2];
    req_kept_base = v[3];
    req_kept = v[4];
    kv_base = v[3] + g[0];
    if (tile == 0 && threadIdx.x == 0) {
      const int64_t gen = a.generated ? a.generated[b] : 0;
      if (a.counts) {
        a.counts[3 * b] = static_cast<int32_t>(v[4]);
        a.counts[3 * b + 1] = static_cast<int32_t>(v[5]);
        a.counts[3 * b + 2] = static_cast<int32_t>(v[6]);
      }
      if (a.kv_indptr) {
        if (b == 0) a.kv_indptr[0] = 0;
        a.kv_indptr[b + 1] = static_cast<int32_t>(kv_base + v[4] + gen);
      }
      if (a.last_page_len) {
        const int64_t len = v[4] + gen;
        a.last_page_len[b] = len > 0 ? static_cast<int32_t>((len - 1) % a.page_size + 1) : 0;
      }
      if (a.status && b + 1 == a.n_requests) {
        // this block's reduction covered every tile of the batch
        const int64_t kept_all = v[3] + v[4];
        // moved and retired over all tiles: those before the last request
        // are the prefix sums of its tile 0 (v[1], v[2])
        const int64_t moved_all = v[1] + v[5];
        const int64_t retired_all = v[2] + v[6];
        const bool bad = moved_all != a.fresh_count || kept_all > a.kept_capacity ||
                         retired_all > a.retired_capacity ||
                         (a.kv_indices && kv_base + v[4] + gen > a.kv_capacity);
        a.status[0] = bad ? 1 : 0;
      }
    }
  } else {
    kv_base = a.req_kv_base[b];
    req_kept = a.req_kept[b];
    req_kept_base = a.tile_offsets[3 * (static_cast<int64_t>(b) * a.tiles_per_req)];
    const int64_t* toff = a.tile_offsets + 3 * (static_cast<int64_t>(b) * a.tiles_per_req + tile);
    carry_kept = toff[0];
    carry_moved = toff[1];
    carry_retired = toff[2];
  }

  // generated raw-row entries after the prompt go after the compacted row
  if (tile == 0 && a.generated && a.kv_indices) {
    const int32_t gen = a.generated[b];
    for (int i = threadIdx.x; i < gen; i += kThreads) {
      const int64_t at = kv_base + req_kept + i;
      if (at < a.kv_capacity) a.kv_indices[at] = row[n + i];
    }
  }
  if (start >= n) return;

  __shared__ int wave_sums[3][kWaves];
  const int w = threadIdx.x >> 6;
  for (int s = 0; s < a.steps; ++s) {
    const int64_t i = start + s * kThreads + threadIdx.x;
    const bool valid = i < n;
    bool kept = false, moved = false;
    int32_t slot = 0, bpos = 0, fpos = 0;
    if (valid) {
      kept = a.keep[base + i] != 0;
      bpos = a.birth[base + i];
      fpos = a.final_pos[base + i];
      moved = kept && bpos != fpos;
      slot = a.birth_slots ? a.birth_slots[base + i] : row[i];
    }
    const bool retired = valid && (!kept || moved);
    const uint64_t mk = __ballot(kept);
    const uint64_t mm = __ballot(moved);
    const uint64_t mr = __ballot(retired);
    if (lane_id() == 0) {
      wave_sums[0][w] = __popcll(mk);
      wave_sums[1][w] = __popcll(mm);
      wave_sums[2][w] = __popcll(mr);
    }
    __syncthreads();
    int64_t pk = carry_kept, pm = carry_moved, pr = carry_retired;
    int tk = 0, tm = 0, tr = 0;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
      if (q < w) {
        pk += wave_sums[0][q];
        pm += wave_sums[1][q];
        pr += wave_sums[2][q];
      }
      tk += wave_sums[0][q];
      tm += wave_sums[1][q];
      tr += wave_sums[2][q];
    }
    pk += rank_below(mk);
    pm += rank_below(mm);
    pr += rank_below(mr);
    if (valid) {
      int32_t terminal = -1;
      if (moved) {
        const int32_t fresh = pm < a.fresh_count ? a.fresh[pm] : -1;
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
        a.raw_indices[pk] = static_cast<int32_t>(i);
        a.active_positions[pk] = fpos;
      }
      if (kept && a.kv_indices) {
        const int64_t at = kv_base + (pk - req_kept_base);
        if (at < a.kv_capacity) a.kv_indices[at] = terminal;
      }
      row[i] = terminal;
    }
    carry_kept += tk;
    carry_moved += tm;
    carry_retired += tr;
    __syncthreads();
  }
}

}  // namespace
}  // namespace akv

extern "C" int64_t akv_compact_workspace_bytes(int32_t n_requests, int64_t max_tokens) {
  using namespace akv;
  if (n_requests < 0 || max_tokens < 0) return -1;
  const int64_t tiles = tiles_per_request(n_requests, max_tokens);
  const int64_t entries = static_cast<int64_t>(n_requests) * tiles;
  // int64 sections first (8-byte aligned), then the int32 tile counts
  return entries * 3 * 8 + static_cast<int64_t>(n_requests) * 16 + entries * 2 * 4;
}

extern "C" int akv_compact_rows(int32_t n_requests, const int64_t* req_offsets, int64_t max_tokens,
                                int32_t* table, int64_t row_stride, const int64_t* row_pointers,
                                const int64_t* req_rows, const uint8_t* keep,
                                const int32_t* birth_positions, const int32_t* final_positions,
                                const int32_t* birth_slots, const int32_t* fresh_slots, int64_t fresh_count, int32_t* retired,
                                int64_t retired_capacity, int32_t* copy_src, int32_t* copy_dst,
                                int32_t* copy_pairs, int32_t* raw_indices,
                                int32_t* active_positions, int64_t kept_capacity,
                                const int32_t* generated, int32_t* kv_indices, int64_t kv_capacity,
                                int32_t* kv_indptr, int32_t* last_page_len, int32_t page_size,
                                int32_t* counts, void* workspace,
                                int64_t workspace_bytes, int32_t* status, void* stream) {
  using namespace akv;
  if (n_requests < 0 || max_tokens < 0)
    return fail(AKV_EINVAL, "akv_compact_rows: negative request or token count");
  if (n_requests == 0) return AKV_OK;
  if (!req_offsets || !req_rows || !keep || !birth_positions || !final_positions || !retired ||
      !copy_src || !copy_dst || !copy_pairs || !raw_indices || !active_positions || !workspace)
    return fail(AKV_EINVAL, "akv_compact_rows: null device pointer");
  if (!row_pointers && !table)
    return fail(AKV_EINVAL, "akv_compact_rows: need a request table or row pointers");
  if (fresh_count > 0 && !fresh_slots)
    return fail(AKV_EINVAL, "akv_compact_rows: fresh_count > 0 with no fresh slots");
  if (last_page_len && page_size <= 0)
    return fail(AKV_EINVAL, "akv_compact_rows: page_size must be positive");
  if (generated && kv_indices && !kv_indptr)
    return fail(AKV_EINVAL, "akv_compact_rows: generated tokens need kv_indptr");
  const int64_t need = akv_compact_workspace_bytes(n_requests, max_tokens);
  if (workspace_bytes < need)
    return fail(AKV_EINVAL, "akv_compact_rows: workspace holds %lld bytes, needs %lld",
                static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  if ((reinterpret_cast<uintptr_t>(workspace) & 7) != 0)
    return fail(AKV_EINVAL, "akv_compact_rows: workspace must be 8-byte aligned");
  const int64_t tiles = tiles_per_request(n_requests, max_tokens);
  if (tiles > 65535 || n_requests > 65535)
    return fail(AKV_EINVAL, "akv_compact_rows: batch too large (%d requests, %lld tiles)", n_requests,
                static_cast<long long>(tiles));
  const int64_t entries = static_cast<int64_t>(n_requests) * tiles;

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
  a.fresh = fresh_slots;
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
  a.tile_offsets = reinterpret_cast<int64_t*>(ws);
  a.req_kv_base = reinterpret_cast<int64_t*>(ws + entries * 3 * 8);
  a.req_kept = a.req_kv_base + n_requests;
  a.tile_counts = reinterpret_cast<int32_t*>(ws + entries * 3 * 8 + static_cast<int64_t>(n_requests) * 16);
  a.n_requests = n_requests;
  a.tiles_per_req = static_cast<int32_t>(tiles);
  a.steps = tile_steps(n_requests, max_tokens);

  hipStream_t st = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(n_requests));
  hipLaunchKernelGGL(compact_count_kernel, grid, dim3(kThreads), 0, st, a);
  int rc = check_launch("akv_compact_rows (count)");
  if (rc) return rc;
  if (entries <= kFusedMaxEntries) {
    hipLaunchKernelGGL(compact_scatter_kernel<true>, grid, dim3(kThreads), 0, st, a);
    return check_launch("akv_compact_rows (scatter)");
  }
  hipLaunchKernelGGL(compact_offsets_kernel, dim3(1), dim3(1024), 0, st, a);
  rc = check_launch("akv_compact_rows (offsets)");
  if (rc) return rc;
  hipLaunchKernelGGL(compact_scatter_kernel<false>, grid, dim3(kThreads), 0, st, a);
  return check_launch("akv_compact_rows (scatter)");
}
