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
// Rows of an even number of 16-byte chunks (up to 2 KiB): a workgroup per
// token with layer rows side by side, double-buffered over the layers (the
// Reposition's structure without the rotation).  Other sizes: flat 16-byte
// work items, kBatch independent loads in flight per thread.
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
      if (dst[k]) *((global_u32x4*)dst[k]) = v[k];
  }
}

// Row-structured variant for rows of an even number of chunks (at most 128):
// a workgroup per token, `rows` layer rows side by side, each lane moving
// chunks j and j + lanes of the K and the V row; the next layer's loads are
// in flight while this layer is stored.
struct RowChunks {
  u32x4 k0, k1, v0, v1;
};

__global__ void __launch_bounds__(1024) copy_kv_rows_vec_kernel(const CopyArgs a, int lanes, int rows) {
  const int64_t t = blockIdx.x;
  const int sub = threadIdx.x / lanes;
  const int j = threadIdx.x - sub * lanes;
  if (sub >= rows || t >= a.n) return;
  const int64_t s = a.src_slots ? a.src_slots[t] : t;
  const int64_t d = a.dst_slots ? a.dst_slots[t] : t;
  auto load = [&](int l) {
    const char* k = reinterpret_cast<const char*>(a.src_k[l]) + s * a.src_k_stride + 16 * j;
    const char* v = reinterpret_cast<const char*>(a.src_v[l]) + s * a.src_v_stride + 16 * j;
    RowChunks r;
    r.k0 = *((const global_u32x4*)k);
    r.k1 = *((const global_u32x4*)(k + 16 * lanes));
    r.v0 = *((const global_u32x4*)v);
    r.v1 = *((const global_u32x4*)(v + 16 * lanes));
    return r;
  };
  auto store = [&](int l, const RowChunks& r) {
    char* k = reinterpret_cast<char*>(a.dst_k[l]) + d * a.dst_k_stride + 16 * j;
    char* v = reinterpret_cast<char*>(a.dst_v[l]) + d * a.dst_v_stride + 16 * j;
    *((global_u32x4*)k) = r.k0;
    *((global_u32x4*)(k + 16 * lanes)) = r.k1;
    *((global_u32x4*)v) = r.v0;
    *((global_u32x4*)(v + 16 * lanes)) = r.v1;
  };
  if (sub >= a.n_layers) return;
  RowChunks cur = load(sub);
  for (int l = sub; l < a.n_layers; l += rows) {
    const int next = l + rows;
    RowChunks nxt = cur;
    if (next < a.n_layers) nxt = load(next);
    store(l, cur);
    cur = nxt;
  }
}

}  // namespace
}  // namespace akv

extern "C" int akv_copy_kv_rows(const uint64_t* src_k_ptrs, const uint64_t* src_v_ptrs, const uint64_t* dst_k_ptrs,
                                const uint64_t* dst_v_ptrs, int32_t n_layers, int64_t row_bytes,
                                int64_t src_k_stride, int64_t src_v_stride, int64_t dst_k_stride,
                                int64_t dst_v_stride, const int32_t* src_slots, const int32_t* dst_slots,
                                int64_t n_tokens, void* stream) {
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
  a.n = n_tokens;
  a.n_layers = n_layers;
  a.chunks = static_cast<int32_t>(row_bytes / 16);
  if (a.chunks % 2 == 0 && a.chunks <= 128) {
    // one workgroup per token, ~192 threads: layer rows side by side,
    // balanced over the passes
    const int lanes = a.chunks / 2;
    int rows = 192 / lanes < 1 ? 1 : 192 / lanes;
    if (rows > n_layers) rows = n_layers;
    const int passes = (n_layers + rows - 1) / rows;
    rows = (n_layers + passes - 1) / passes;
    if (n_tokens > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_copy_kv_rows: too many tokens");
    hipLaunchKernelGGL(copy_kv_rows_vec_kernel, dim3(static_cast<unsigned>(n_tokens)), dim3(lanes * rows), 0,
                       as_stream(stream), a, lanes, rows);
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
