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
// Work item = one 16-byte chunk; a workgroup takes kTokens tokens x all
// layers x {K, V} x row chunks and keeps kBatch independent loads in
// flight per thread before storing them.
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
  // about 16 chunks per thread per workgroup
  const int64_t per_token = static_cast<int64_t>(n_layers) * 2 * a.chunks;
  int64_t tokens = (static_cast<int64_t>(kThreads) * 16 + per_token - 1) / per_token;
  a.tokens_per_block = static_cast<int32_t>(tokens < 1 ? 1 : (tokens > 4096 ? 4096 : tokens));
  const int64_t blocks = (n_tokens + a.tokens_per_block - 1) / a.tokens_per_block;
  if (blocks > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_copy_kv_rows: too many tokens");
  hipLaunchKernelGGL(copy_kv_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, as_stream(stream),
                     a);
  return check_launch("akv_copy_kv_rows");
}
