// Occurrence binding of a fresh request's whole-prompt forward (gfx950).
//
// Given the occurrence window of a multi-stage program (every (raw token,
// position) version a segment reads, plus the terminal versions), binds
// physical slots the way plan_occurrence_materialization + OccurrenceState
// .advance do for query_start = 0, query_end = n with every slot request-owned
// (akv/system/sglang/srt/context_system/occurrence.py:341-466, 632-755):
//   required  = birth versions, versions a segment reads (ids < first_final),
//               and terminal versions of kept tokens;
//   reuse     = the version's position equals the token's birth position
//               (it is the birth slot, no copy);
//   allocated = required non-birth versions that are not reused: they take
//               the fresh slots in occurrence order and are copied from the
//               birth slot with pair (birth position, version position);
//   terminal row = kept ? slot of the terminal version : -1;
//   retired   = birth slots that are not terminal (raw order), then fresh
//               slots that are not terminal (allocation order).
// Two launches, no inter-workgroup waiting: per-tile counts, then a scatter
// whose workgroups derive their offsets from the earlier tiles' counts.
#include "common.h"

namespace akv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSteps = 16;

int bind_steps(int32_t n_requests, int64_t max_count) {
  const int64_t work = static_cast<int64_t>(n_requests) * max_count;
  int steps = 1;
  while (steps < kMaxSteps && work > static_cast<int64_t>(kThreads) * steps * 1024) steps <<= 1;
  return steps;
}

int64_t bind_tiles(int32_t n_requests, int64_t max_count) {
  const int64_t tile = static_cast<int64_t>(kThreads) * bind_steps(n_requests, max_count);
  return max_count <= 0 ? 1 : (max_count + tile - 1) / tile;
}

struct BindArgs {
  // bases[k * (B + 1) + b]: k = 0 occurrence offsets, 1 raw offsets, 2 copy
  // offsets, 3 retired offsets, 4 start of the fresh part of b's retired list,
  // 5 first_final (request-local occurrence id)
  const int64_t* bases;
  const int32_t* occ_raw;       // request-local raw index per occurrence
  const int32_t* occ_pos;
  const int32_t* terminal_occ;  // request-local occurrence id per raw token
  const uint8_t* keep;
  const int32_t* birth_slots;   // per raw token
  const int32_t* fresh_slots;   // per allocated occurrence
  int32_t* occ_slots;
  int32_t* copy_src;
  int32_t* copy_dst;
  int32_t* copy_pairs;
  int32_t* retired;
  int32_t* table;
  int64_t row_stride;
  const int64_t* row_pointers;
  const int64_t* req_rows;
  int32_t* tile_counts;  // [B][tiles][3] allocated, fresh retired, birth retired
  int32_t n_requests;
  int32_t tiles;
  int32_t steps;
};

struct Flags {
  bool alloc, fresh_retired, birth_retired;
};

struct Occ {
  int64_t c;  // request-local occurrence id
  int32_t raw, pos, birth_pos;
  bool birth, reuse, required, terminal_live;
};

__device__ __forceinline__ const int64_t* row(const BindArgs& a, int k) { return a.bases + k * (a.n_requests + 1); }

__device__ __forceinline__ Occ describe(const BindArgs& a, int b, int64_t c) {
  const int64_t ob = row(a, 0)[b], rb = row(a, 1)[b];
  const int64_t n = row(a, 1)[b + 1] - rb;
  Occ o;
  o.c = c;
  o.raw = a.occ_raw[ob + c];
  o.pos = a.occ_pos[ob + c];
  o.birth_pos = a.occ_pos[ob + o.raw];  // occurrence id raw is the birth version
  o.birth = c < n;
  o.reuse = o.pos == o.birth_pos;
  const bool kept = a.keep[rb + o.raw] != 0;
  o.required = o.birth || c < row(a, 5)[b] || kept;
  o.terminal_live = kept && a.terminal_occ[rb + o.raw] == c;
  return o;
}

__device__ __forceinline__ Flags flags_of(const BindArgs& a, int b, const Occ& o) {
  Flags f;
  f.alloc = !o.birth && o.required && !o.reuse;
  f.fresh_retired = f.alloc && !o.terminal_live;
  f.birth_retired = false;
  if (o.birth) {
    // the birth slot stays live when the token is kept and its terminal
    // version sits at the birth position
    const int64_t ob = row(a, 0)[b], rb = row(a, 1)[b];
    const bool kept = a.keep[rb + o.raw] != 0;
    const int32_t t = a.terminal_occ[rb + o.raw];
    f.birth_retired = !(kept && a.occ_pos[ob + t] == o.birth_pos);
  }
  return f;
}

__device__ __forceinline__ int rank_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

__global__ void __launch_bounds__(kThreads) bind_count_kernel(const BindArgs a) {
  const int b = blockIdx.y;
  const int tile = blockIdx.x;
  const int64_t count = row(a, 0)[b + 1] - row(a, 0)[b];
  const int64_t start = static_cast<int64_t>(tile) * kThreads * a.steps;
  int v[3] = {0, 0, 0};
  for (int s = 0; s < a.steps; ++s) {
    const int64_t c = start + s * kThreads + threadIdx.x;
    if (c < count) {
      const Flags f = flags_of(a, b, describe(a, b, c));
      v[0] += f.alloc;
      v[1] += f.fresh_retired;
      v[2] += f.birth_retired;
    }
  }
  __shared__ int sums[kWaves][3];
#pragma unroll
  for (int k = 0; k < 3; ++k)
    for (int off = 32; off > 0; off >>= 1) v[k] += __shfl_xor(v[k], off);
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int k = 0; k < 3; ++k) sums[threadIdx.x >> 6][k] = v[k];
  __syncthreads();
  if (threadIdx.x < 3) {
    int t = 0;
    for (int w = 0; w < kWaves; ++w) t += sums[w][threadIdx.x];
    a.tile_counts[(static_cast<int64_t>(b) * a.tiles + tile) * 3 + threadIdx.x] = t;
  }
}

__global__ void __launch_bounds__(kThreads) bind_scatter_kernel(const BindArgs a) {
  const int b = blockIdx.y;
  const int tile = blockIdx.x;
  const int64_t ob = row(a, 0)[b], rb = row(a, 1)[b];
  const int64_t count = row(a, 0)[b + 1] - ob;
  const int64_t start = static_cast<int64_t>(tile) * kThreads * a.steps;
  if (start >= count) return;
  // this tile's offsets: the earlier tiles' counts of the request
  __shared__ int64_t red[kWaves][3];
  __shared__ int64_t carry[3];
  int64_t v[3] = {0, 0, 0};
  for (int t = threadIdx.x; t < tile; t += kThreads)
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] += a.tile_counts[(static_cast<int64_t>(b) * a.tiles + t) * 3 + k];
#pragma unroll
  for (int k = 0; k < 3; ++k)
    for (int off = 32; off > 0; off >>= 1) v[k] += __shfl_xor(v[k], off);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int k = 0; k < 3; ++k) red[w][k] = v[k];
  __syncthreads();
  if (threadIdx.x < 3) {
    int64_t t = 0;
    for (int q = 0; q < kWaves; ++q) t += red[q][threadIdx.x];
    carry[threadIdx.x] = t;
  }
  __syncthreads();
  const int64_t copy_lo = row(a, 2)[b], copy_hi = row(a, 2)[b + 1];
  const int64_t ret_lo = row(a, 3)[b], ret_hi = row(a, 3)[b + 1];
  const int64_t fresh_ret_lo = row(a, 4)[b];
  int32_t* trow = a.row_pointers ? reinterpret_cast<int32_t*>(a.row_pointers[a.req_rows[b]])
                                 : a.table + a.req_rows[b] * a.row_stride;
  __shared__ int wave_tot[kWaves][3];
  for (int s = 0; s < a.steps; ++s) {
    const int64_t c = start + s * kThreads + threadIdx.x;
    const bool in = c < count;
    Occ o{};
    Flags f{false, false, false};
    if (in) {
      o = describe(a, b, c);
      f = flags_of(a, b, o);
    }
    const uint64_t m0 = __ballot(f.alloc), m1 = __ballot(f.fresh_retired), m2 = __ballot(f.birth_retired);
    if ((threadIdx.x & 63) == 0) {
      wave_tot[w][0] = __popcll(m0);
      wave_tot[w][1] = __popcll(m1);
      wave_tot[w][2] = __popcll(m2);
    }
    __syncthreads();
    int64_t r[3] = {carry[0], carry[1], carry[2]};
    for (int q = 0; q < w; ++q)
#pragma unroll
      for (int k = 0; k < 3; ++k) r[k] += wave_tot[q][k];
    r[0] += rank_below(m0);
    r[1] += rank_below(m1);
    r[2] += rank_below(m2);
    if (in) {
      const int32_t birth_slot = a.birth_slots[rb + o.raw];
      int32_t slot = -1;
      if (f.alloc) {
        const int64_t at = copy_lo + r[0];
        if (at < copy_hi) {
          slot = a.fresh_slots[at];
          a.copy_src[at] = birth_slot;
          a.copy_dst[at] = slot;
          a.copy_pairs[2 * at] = o.birth_pos;
          a.copy_pairs[2 * at + 1] = o.pos;
        }
        if (f.fresh_retired) {
          const int64_t rt = fresh_ret_lo + r[1];
          if (rt < ret_hi) a.retired[rt] = slot;
        }
      } else if (o.birth || o.required) {
        slot = birth_slot;
      }
      a.occ_slots[ob + c] = slot;
      if (f.birth_retired) {
        const int64_t rt = ret_lo + r[2];
        if (rt < fresh_ret_lo) a.retired[rt] = birth_slot;
      }
      // terminal row: the terminal version of a kept token writes its slot,
      // the birth version of a dropped token writes the hole
      if (o.terminal_live) trow[o.raw] = slot;
      if (o.birth && a.keep[rb + o.raw] == 0) trow[o.raw] = -1;
    }
    __syncthreads();
    if (threadIdx.x < 3) {
      int64_t t = 0;
      for (int q = 0; q < kWaves; ++q) t += wave_tot[q][threadIdx.x];
      carry[threadIdx.x] += t;
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace akv

extern "C" int64_t akv_bind_workspace_bytes(int32_t n_requests, int64_t max_occurrences) {
  using namespace akv;
  if (n_requests < 0 || max_occurrences < 0) return -1;
  return static_cast<int64_t>(n_requests) * bind_tiles(n_requests, max_occurrences) * 3 * 4;
}

extern "C" int akv_bind_occurrences(int32_t n_requests, const int64_t* bases, int64_t max_occurrences,
                                    const int32_t* occurrence_raw_tokens, const int32_t* occurrence_positions,
                                    const int32_t* terminal_occurrences, const uint8_t* keep,
                                    const int32_t* birth_slots, const int32_t* fresh_slots,
                                    int32_t* occurrence_slots, int32_t* copy_src, int32_t* copy_dst,
                                    int32_t* copy_pairs, int32_t* retired, int32_t* table, int64_t row_stride,
                                    const int64_t* row_pointers, const int64_t* req_rows, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  using namespace akv;
  if (n_requests < 0 || max_occurrences < 0) return fail(AKV_EINVAL, "akv_bind_occurrences: negative size");
  if (n_requests == 0 || max_occurrences == 0) return AKV_OK;
  if (!bases || !occurrence_raw_tokens || !occurrence_positions || !terminal_occurrences || !keep ||
      !birth_slots || !occurrence_slots || !copy_src || !copy_dst || !copy_pairs || !retired || !req_rows ||
      !workspace)
    return fail(AKV_EINVAL, "akv_bind_occurrences: null device pointer");
  if (!row_pointers && !table) return fail(AKV_EINVAL, "akv_bind_occurrences: need a request table or row pointers");
  if (n_requests > 65535) return fail(AKV_EINVAL, "akv_bind_occurrences: batch too large");
  const int64_t need = akv_bind_workspace_bytes(n_requests, max_occurrences);
  if (workspace_bytes < need)
    return fail(AKV_EINVAL, "akv_bind_occurrences: workspace holds %lld bytes, needs %lld",
                static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  BindArgs a{};
  a.bases = bases;
  a.occ_raw = occurrence_raw_tokens;
  a.occ_pos = occurrence_positions;
  a.terminal_occ = terminal_occurrences;
  a.keep = keep;
  a.birth_slots = birth_slots;
  a.fresh_slots = fresh_slots;
  a.occ_slots = occurrence_slots;
  a.copy_src = copy_src;
  a.copy_dst = copy_dst;
  a.copy_pairs = copy_pairs;
  a.retired = retired;
  a.table = table;
  a.row_stride = row_stride;
  a.row_pointers = row_pointers;
  a.req_rows = req_rows;
  a.tile_counts = static_cast<int32_t*>(workspace);
  a.n_requests = n_requests;
  a.steps = bind_steps(n_requests, max_occurrences);
  const int64_t tiles = bind_tiles(n_requests, max_occurrences);
  if (tiles > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_bind_occurrences: window too large");
  a.tiles = static_cast<int32_t>(tiles);
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(n_requests));
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(bind_count_kernel, grid, dim3(kThreads), 0, st, a);
  int rc = check_launch("akv_bind_occurrences (count)");
  if (rc) return rc;
  hipLaunchKernelGGL(bind_scatter_kernel, grid, dim3(kThreads), 0, st, a);
  return check_launch("akv_bind_occurrences (scatter)");
}
