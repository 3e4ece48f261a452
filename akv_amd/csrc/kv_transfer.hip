// All-layer KV row copy between two slot spaces (gfx950): the compacted
// final-version handoff of a Context request.
//
// For token t and layer l, the K row and the V row (H * D contiguous
// elements, `row_bytes` each) at slot src_slots[t] of the source layer
// buffers are copied to slot dst_slots[t] of the destination layer buffers.
// Either side may be a pool (slot = a request's active slot) or a packed
// buffer (slot = t, slots pointer NULL), so one kernel is the P-side pack of
// request_active_slots, the D-side unpack into freshly allocated owners
// (akv/system/sglang/srt/disaggregation/context_transfer.py:110-128,
// 201-259), and a direct pool-to-pool copy -- to a peer GPU's pool when the
// destination pointers are peer (xGMI) addresses.
//
// Rows of up to 8 KiB: one wave per row (several rows per wave when a row is
// under 1 KiB), rows numbered layer-major -- (layer, K/V) outermost, token
// innermost -- so the whole grid sweeps one layer's buffers at a time.  On
// MI355X this measured ~4% faster than a workgroup per token walking its
// layers, for the same random 1 KiB rows; with no slot vectors on either
// side it is a streaming copy.  Longer rows: flat 16-byte work items,
// kBatch independent loads in flight per thread.  Stores are nontemporal (a
// copied row is not read back here): on MI355X the pack measured +8%, the
// unpack and pool-to-pool copies +2%, the random-row gather +1.5-2% and the
// streaming copy +3% against plain stores.
#include "common.h"

namespace akv {
namespace {

constexpr int kThreads = 256;
constexpr int kBatch = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4 global_u32x4;

struct CopyArgs {
  const uint64_t* src_k;
  const uint64_t* src_v;
  const uint64_t* dst_k;
  const uint64_t* dst_v;
  int64_t src_k_stride, src_v_stride, dst_k_stride, dst_v_stride;  // bytes between slots
  const int32_t* src_slots;
  const int32_t* dst_slots;
  const int32_t* gate;  // compaction status word, or nullptr
  int64_t n;
  int32_t n_layers;
  int32_t chunks;  // 16-byte chunks per row
  int32_t tokens_per_block;
};

__global__ void __launch_bounds__(kThreads) copy_kv_rows_kernel(const CopyArgs a) {
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * a.tokens_per_block;
  const int64_t per_token = static_cast<int64_t>(a.n_layers) * 2 * a.chunks;
  const int64_t tokens = a.n - t0 < a.tokens_per_block ? a.n - t0 : a.tokens_per_block;
  const int64_t items = tokens * per_token;
  if (gated(a.gate)) return;
  for (int64_t base = 0; base < items; base += static_cast<int64_t>(kThreads) * kBatch) {
    u32x4 v[kBatch];
    char* dst[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int64_t w = base + static_cast<int64_t>(k) * kThreads + threadIdx.x;
      dst[k] = nullptr;
      if (w < items) {
        const int64_t t = t0 + w / per_token;
        int64_t r = w % per_token;
        const int c = static_cast<int>(r % a.chunks);
        r /= a.chunks;
        const int kv = static_cast<int>(r & 1);
        const int l = static_cast<int>(r >> 1);
        const int64_t s = a.src_slots ? a.src_slots[t] : t;
        const int64_t d = a.dst_slots ? a.dst_slots[t] : t;
        const char* src = reinterpret_cast<const char*>(kv ? a.src_v[l] : a.src_k[l]) +
                          s * (kv ? a.src_v_stride : a.src_k_stride) + 16 * c;
        dst[k] = reinterpret_cast<char*>(kv ? a.dst_v[l] : a.dst_k[l]) + d * (kv ? a.dst_v_stride : a.dst_k_stride) +
                 16 * c;
        v[k] = *((const global_u32x4*)src);
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (dst[k]) __builtin_nontemporal_store(v[k], (global_u32x4*)dst[k]);
  }
}

// Layer-major row copy: grid (token blocks, layers x {K, V}) -- blocks are
// dispatched x fastest, so the grid sweeps one layer's K (then V) rows before
// the next layer's.  2^shift lanes per row (at most 64), 64 >> shift rows per
// wave, each lane moving chunks c, c + lanes, ... (at most U): all loads,
// then all stores.  No division anywhere.  SRC / DST: the side has a slot
// vector (a compile-time choice: a branch on the pointer measured 2.5%
// slower).
template <int U, bool SRC, bool DST>
__global__ void __launch_bounds__(256) copy_rows_layer_major(const CopyArgs a, int shift) {
  const int lane = threadIdx.x & 63;
  const int lanes = 1 << shift;
  const int c0 = lane & (lanes - 1);
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t t = (wave << (6 - shift)) + (lane >> shift);
  if (t >= a.n) return;
  const int l = static_cast<int>(blockIdx.y >> 1);
  const bool kv = blockIdx.y & 1;
  const int64_t s = SRC ? static_cast<int64_t>(a.src_slots[t]) : t;
  const int64_t d = DST ? static_cast<int64_t>(a.dst_slots[t]) : t;
  // the gate is read with the slot entries and closes before the rows
  if (gated(a.gate)) return;
  const char* src = reinterpret_cast<const char*>(kv ? a.src_v[l] : a.src_k[l]) + s * (kv ? a.src_v_stride : a.src_k_stride);
  char* dst = reinterpret_cast<char*>(kv ? a.dst_v[l] : a.dst_k[l]) + d * (kv ? a.dst_v_stride : a.dst_k_stride);
  u32x4 v[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int c = c0 + k * lanes;
    if (c < a.chunks) v[k] = *((const global_u32x4*)(src + 16 * c));
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int c = c0 + k * lanes;
    if (c < a.chunks) __builtin_nontemporal_store(v[k], (global_u32x4*)(dst + 16 * c));
  }
}

template <int U>
void launch_sides(int sides, dim3 grid, hipStream_t st, const CopyArgs& a, int shift) {
  switch (sides) {
    case 3:
      hipLaunchKernelGGL((copy_rows_layer_major<U, true, true>), grid, dim3(256), 0, st, a, shift);
      break;
    case 2:
      hipLaunchKernelGGL((copy_rows_layer_major<U, true, false>), grid, dim3(256), 0, st, a, shift);
      break;
    case 1:
      hipLaunchKernelGGL((copy_rows_layer_major<U, false, true>), grid, dim3(256), 0, st, a, shift);
      break;
    default:
      hipLaunchKernelGGL((copy_rows_layer_major<U, false, false>), grid, dim3(256), 0, st, a, shift);
  }
}

void launch_layer_major(int u, int sides, dim3 grid, hipStream_t st, const CopyArgs& a, int shift) {
  if (u == 1)
    launch_sides<1>(sides, grid, st, a, shift);
  else if (u == 2)
    launch_sides<2>(sides, grid, st, a, shift);
  else if (u == 4)
    launch_sides<4>(sides, grid, st, a, shift);
  else
    launch_sides<8>(sides, grid, st, a, shift);
}

}  // namespace
}  // namespace akv

extern "C" int akv_copy_kv_rows(const uint64_t* src_k_ptrs, const uint64_t* src_v_ptrs, const uint64_t* dst_k_ptrs,
                                const uint64_t* dst_v_ptrs, int32_t n_layers, int64_t row_bytes,
                                int64_t src_k_stride, int64_t src_v_stride, int64_t dst_k_stride,
                                int64_t dst_v_stride, const int32_t* src_slots, const int32_t* dst_slots,
                                int64_t n_tokens, const int32_t* status, void* stream) {
  using namespace akv;
  if (n_layers < 0 || n_tokens < 0) return fail(AKV_EINVAL, "akv_copy_kv_rows: negative size");
  if (n_layers == 0 || n_tokens == 0) return AKV_OK;
  if (!src_k_ptrs || !src_v_ptrs || !dst_k_ptrs || !dst_v_ptrs)
    return fail(AKV_EINVAL, "akv_copy_kv_rows: null pointer table");
  if (row_bytes <= 0 || row_bytes % 16 != 0 || row_bytes / 16 > 0x7fffffff)
    return fail(AKV_EINVAL, "akv_copy_kv_rows: row_bytes must be a positive multiple of 16");
  if ((src_k_stride | src_v_stride | dst_k_stride | dst_v_stride) % 16 != 0 || src_k_stride < row_bytes ||
      src_v_stride < row_bytes || dst_k_stride < row_bytes || dst_v_stride < row_bytes)
    return fail(AKV_EINVAL, "akv_copy_kv_rows: slot strides must be multiples of 16 bytes covering a row");
  CopyArgs a{};
  a.src_k = src_k_ptrs;
  a.src_v = src_v_ptrs;
  a.dst_k = dst_k_ptrs;
  a.dst_v = dst_v_ptrs;
  a.src_k_stride = src_k_stride;
  a.src_v_stride = src_v_stride;
  a.dst_k_stride = dst_k_stride;
  a.dst_v_stride = dst_v_stride;
  a.src_slots = src_slots;
  a.dst_slots = dst_slots;
  a.gate = status;
  a.n = n_tokens;
  a.n_layers = n_layers;
  a.chunks = static_cast<int32_t>(row_bytes / 16);
  if (a.chunks <= 512 && n_layers <= 32767) {
    // lanes per row: the power of two covering the row, at most a wave
    int shift = 0;
    while ((1 << shift) < a.chunks && shift < 6) ++shift;
    const int lanes = 1 << shift;
    const int per_lane = (a.chunks + lanes - 1) / lanes;
    const int64_t waves = (n_tokens + (64 >> shift) - 1) >> (6 - shift);
    const int64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_copy_kv_rows: too many tokens");
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(2 * n_layers));
    hipStream_t st = as_stream(stream);
    const int u = per_lane == 1 ? 1 : per_lane == 2 ? 2 : per_lane <= 4 ? 4 : 8;
    const int sides = (src_slots ? 2 : 0) + (dst_slots ? 1 : 0);
    launch_layer_major(u, sides, grid, st, a, shift);
    return check_launch("akv_copy_kv_rows");
  }
  // any other row size: flat 16-byte work items, about 16 per thread
  const int64_t per_token = static_cast<int64_t>(n_layers) * 2 * a.chunks;
  int64_t tokens = (static_cast<int64_t>(kThreads) * 16 + per_token - 1) / per_token;
  a.tokens_per_block = static_cast<int32_t>(tokens < 1 ? 1 : (tokens > 4096 ? 4096 : tokens));
  const int64_t blocks = (n_tokens + a.tokens_per_block - 1) / a.tokens_per_block;
  if (blocks > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_copy_kv_rows: too many tokens");
  hipLaunchKernelGGL(copy_kv_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, as_stream(stream),
                     a);
  return check_launch("akv_copy_kv_rows");
}
