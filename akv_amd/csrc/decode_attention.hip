// GQA decode attention with attention sinks over compacted page-one indices
// (gfx950, MFMA).  The consumer of the Drop + Reposition metadata: one decode
// step reads each request's keys through kv_indptr / kv_indices (full layers)
// or the window-limited indices (sliding-window layers) and normalises with a
// per-head sink logit:
//   o_h = sum_j exp(s_hj) v_j / (sum_j exp(s_hj) + exp(sink_h)),
//   s_hj = scale * q_h . k_j
// which equals the reference's o * sigmoid(lse - sink)
// (akv/system/sglang/srt/layers/attention/context_backend.py:254-272).
//
// Split-K: workgroup = one wave = (chunk of kChunk keys, KV head, request).
// Per 16-key tile:  S^T[16 keys x 16 heads] = K[16 x D] . Q^T[D x 16] on
// v_mfma_f32_16x16x16_bf16 (the group's q heads padded to 16 rows), online
// softmax per head (column), then O^T[D x 16] += V^T[D x 16] . P^T[16 x 16]
// where P^T is already in the B-operand layout of the second MFMA (no
// shuffle) and V goes through LDS to be read transposed.  A combine kernel
// merges the chunks and the sink; when every request fits one chunk (a
// sliding-window layer) the partial kernel applies the sink itself and the
// combine is not launched.
//
// MFMA 16x16x16 bf16 lane layout (verified on gfx950): lane l supplies
// A[l%16][4(l/16)+i] and B[4(l/16)+i][l%16] and holds D[4(l/16)+i][l%16].
#include <cmath>

#include <mutex>

#include "common.h"

namespace akv {
namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4 global_u32x4;

constexpr int kChunk = 256;  // keys per workgroup
constexpr int kTile = 16;    // keys per MFMA tile
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const __bf16* q;
  int64_t q_stride_b, q_stride_h;
  const __bf16* k;
  const __bf16* v;
  int64_t k_stride_slot, k_stride_head, v_stride_slot, v_stride_head;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const float* sinks;
  const int32_t* gate;  // compaction status word, or nullptr
  float scale_log2;  // scale * log2(e)
  void* out;
  int32_t out_f32;
  int64_t out_stride_b, out_stride_h;
  int32_t n_requests, q_heads, kv_heads, group, chunks;
  float* partial;  // [B][Hkv][chunks][16][D + 2]  (o..., m, l)
};

__device__ __forceinline__ short bf16_bits(float x) {
  return __builtin_bit_cast(short, static_cast<__bf16>(x));
}

// Workgroup = one wave = (chunk of kChunk keys, KV head, request).  (Putting
// all KV heads of a chunk in one workgroup, so key rows are read whole,
// measured slower: the per-tile barrier then couples 8 waves.)
template <int D>
__global__ void __launch_bounds__(64) decode_attention_partial_kernel(const AttnArgs a) {
  constexpr int kSteps = D / 16;    // MFMA k-steps over the head dim
  constexpr int kPer = D / 4;       // dims per lane for the K operand
  __shared__ __attribute__((aligned(16))) __bf16 vtile[kTile][D];

  const int lane = threadIdx.x;
  const int chunk = blockIdx.x;
  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int64_t begin = a.kv_indptr[b];
  const int64_t len = a.kv_indptr[b + 1] - begin;
  // a closed gate stops the workgroup before its key indices and rows
  if (gated(a.gate)) return;
  const int64_t c0 = static_cast<int64_t>(chunk) * kChunk;
  float* part = a.partial + ((static_cast<int64_t>(b) * a.kv_heads + g) * a.chunks + chunk) * 16 * (D + 2);
  const int col = lane & 15;   // head within the group (B / D layout column)
  const int quad = lane >> 4;  // 0..3
  if (c0 >= len) {
    if (a.chunks == 1) {
      // one chunk and no keys: the output is 0, sink or not (no combine runs)
      if (col < a.group) {
        const int64_t at = static_cast<int64_t>(b) * a.out_stride_b +
                           static_cast<int64_t>(g * a.group + col) * a.out_stride_h;
#pragma unroll
        for (int t = 0; t < D / 16; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d = 16 * t + 4 * quad + i;
            if (a.out_f32)
              static_cast<float*>(a.out)[at + d] = 0.f;
            else
              static_cast<__bf16*>(a.out)[at + d] = static_cast<__bf16>(0.f);
          }
      }
      return;
    }
    // empty chunk: neutral partial (m = -inf, l = 0)
    if (quad == 0) {
      part[col * (D + 2) + D] = -INFINITY;
      part[col * (D + 2) + D + 1] = 0.f;
    }
    return;
  }
  const int64_t c1 = c0 + kChunk < len ? c0 + kChunk : len;

  // Q^T operand: lane supplies q[head col][dims quad*kPer + 4s + i]
  s16x4 qop[kSteps];
  {
    const bool live = col < a.group;
    const __bf16* qrow = a.q + static_cast<int64_t>(b) * a.q_stride_b +
                         static_cast<int64_t>(g * a.group + (live ? col : 0)) * a.q_stride_h + quad * kPer;
#pragma unroll
    for (int s = 0; s < kSteps; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) qop[s][i] = live ? __builtin_bit_cast(short, qrow[4 * s + i]) : short(0);
  }

  f32x4 acc[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // Registers of one 16-key tile between its global loads and its use.
  constexpr int kVUnits = kTile * D / 8 / 64;  // 16-byte V units per lane
  struct Tile {
    u32x4 k[kPer / 8];
    u32x4 v[kVUnits];
  };
  auto load_tile = [&](int64_t t0) {
    Tile r;
    // this lane's key for the K operand / slot lookup: key t0 + col
    const bool valid = t0 + col < c1;
    const int32_t slot = valid ? a.kv_indices[begin + t0 + col] : 0;
    const __bf16* krow =
        a.k + static_cast<int64_t>(slot) * a.k_stride_slot + static_cast<int64_t>(g) * a.k_stride_head + quad * kPer;
#pragma unroll
    for (int q8 = 0; q8 < kPer / 8; ++q8)
      r.k[q8] = valid ? *((const global_u32x4*)(krow + 8 * q8)) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int q8 = 0; q8 < kVUnits; ++q8) {
      const int u = lane + 64 * q8;
      const int key = u / (D / 8);
      const int part8 = u - key * (D / 8);
      const int32_t ks = __shfl(slot, key);
      r.v[q8] = t0 + key < c1 ? *((const global_u32x4*)(a.v + static_cast<int64_t>(ks) * a.v_stride_slot +
                                                        static_cast<int64_t>(g) * a.v_stride_head + part8 * 8))
                              : u32x4{0u, 0u, 0u, 0u};
    }
    return r;
  };

  // Software-pipelined: the next tile's K and V loads are in flight while
  // this tile's MFMAs and softmax run.
  Tile cur = load_tile(c0);
  for (int64_t t0 = c0; t0 < c1; t0 += kTile) {
    Tile nxt = cur;
    if (t0 + kTile < c1) nxt = load_tile(t0 + kTile);
    // ---- S^T = K . Q^T
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      // dims quad*kPer + 4*st .. +3 live in k[st / 2], words (st % 2) * 2 .. +1
      const u32x4 w = cur.k[st >> 1];
      const uint32_t lo = (st & 1) ? w.z : w.x;
      const uint32_t hi = (st & 1) ? w.w : w.y;
      s16x4 kop;
      kop[0] = static_cast<short>(lo & 0xffff);
      kop[1] = static_cast<short>(lo >> 16);
      kop[2] = static_cast<short>(hi & 0xffff);
      kop[3] = static_cast<short>(hi >> 16);
      s = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(kop, qop[st], s, 0, 0, 0);
    }
    // lane holds S^T[keys t0 + 4*quad + i][head col]
    float p[4];
    float tile_max = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = t0 + 4 * quad + i < c1;
      p[i] = ok ? s[i] * a.scale_log2 : -INFINITY;
      tile_max = fmaxf(tile_max, p[i]);
    }
    tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16));
    tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
    const float m_new = fmaxf(m_run, tile_max);
    const float corr = m_new == -INFINITY ? 1.f : exp2f(m_run - m_new);
    float row = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = m_new == -INFINITY ? 0.f : exp2f(p[i] - m_new);
      row += p[i];
    }
    row += __shfl_xor(row, 16);
    row += __shfl_xor(row, 32);
    l_run = l_run * corr + row;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) acc[t] *= corr;

    // ---- V tile -> LDS (16 keys x D); rows past the chunk were loaded as 0
#pragma unroll
    for (int q8 = 0; q8 < kVUnits; ++q8) {
      const int u = lane + 64 * q8;
      const int key = u / (D / 8);
      *reinterpret_cast<u32x4*>(&vtile[key][(u - key * (D / 8)) * 8]) = cur.v[q8];
    }
    __syncthreads();
    // ---- O^T += V^T . P^T ; P^T is this lane's B operand as is
    s16x4 pop;
#pragma unroll
    for (int i = 0; i < 4; ++i) pop[i] = bf16_bits(p[i]);
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      s16x4 vop;
#pragma unroll
      for (int i = 0; i < 4; ++i) vop[i] = __builtin_bit_cast(short, vtile[4 * quad + i][16 * t + col]);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vop, pop, acc[t], 0, 0, 0);
    }
    __syncthreads();
    cur = nxt;
  }
  // lane holds O^T[dims 16t + 4*quad + i][head col]; every lane of a column
  // carries that head's m and l
  if (a.chunks == 1) {
    // one chunk holds every key: normalise with the sink here (the combine's
    // arithmetic for a single partial) and skip the combine launch
    if (col < a.group) {
      const int h = g * a.group + col;
      const float sink = a.sinks ? a.sinks[h] * kLog2e : -INFINITY;
      const bool valid = m_run != -INFINITY;
      const float mt = valid ? fmaxf(sink, m_run) : sink;
      float lt = (a.sinks && mt != -INFINITY) ? exp2f(sink - mt) : 0.f;
      const float sw = valid ? exp2f(m_run - mt) : 0.f;
      lt += valid ? l_run * sw : 0.f;
      const int64_t at = static_cast<int64_t>(b) * a.out_stride_b + static_cast<int64_t>(h) * a.out_stride_h;
#pragma unroll
      for (int t = 0; t < D / 16; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ot = valid ? acc[t][i] * sw : 0.f;
          const float r = lt > 0.f ? ot / lt : 0.f;
          const int d = 16 * t + 4 * quad + i;
          if (a.out_f32)
            static_cast<float*>(a.out)[at + d] = r;
          else
            static_cast<__bf16*>(a.out)[at + d] = static_cast<__bf16>(r);
        }
    }
    return;
  }
  if (col < a.group) {
    float* ph = part + col * (D + 2);
#pragma unroll
    for (int t = 0; t < D / 16; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) ph[16 * t + 4 * quad + i] = acc[t][i];
    if (quad == 0) {
      ph[D] = m_run;
      ph[D + 1] = l_run;
    }
  }
}

// One workgroup per (request, q head): merge chunk partials and the sink.
// kCombineThreads threads in ways of D / 4 lanes (four dims per lane: two
// 8-byte loads per chunk, as a partial row of D + 2 floats is 8-byte
// aligned); each way folds every ways-th chunk with an online
// (max, sum) merge -- the loads of one chunk do not wait on the previous
// one -- and the ways meet in LDS.
constexpr int kCombineThreads = 256;

template <int D>
__global__ void __launch_bounds__(kCombineThreads) decode_attention_combine_kernel(const AttnArgs a) {
  constexpr int kLanes = D / 4;
  constexpr int kWays = kCombineThreads / kLanes;
  __shared__ float s_m[kWays], s_l[kWays];
  __shared__ __attribute__((aligned(16))) float s_o[kWays][D];
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int g = h / a.group;
  const int hl = h - g * a.group;
  const int dl = threadIdx.x % kLanes;
  const int way = threadIdx.x / kLanes;
  const int64_t len = a.kv_indptr[b + 1] - a.kv_indptr[b];
  if (gated(a.gate)) return;
  // keys past max_len (a caller error) are not read: the partials stop there
  const int64_t want = (len + kChunk - 1) / kChunk;
  const int used = static_cast<int>(want < a.chunks ? want : a.chunks);
  const float* base = a.partial + (static_cast<int64_t>(b) * a.kv_heads + g) * a.chunks * 16 * (D + 2);
  float m = -INFINITY, l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int c = way; c < used; c += kWays) {
    const float* pc = base + (c * 16 + hl) * (D + 2);
    const float mc = pc[D];
    const float lc = pc[D + 1];
    // a partial row is D + 2 floats: 8-byte aligned, so two 8-byte loads
    const f32x2_t lo = *reinterpret_cast<const f32x2_t*>(pc + 4 * dl);
    const f32x2_t hi = *reinterpret_cast<const f32x2_t*>(pc + 4 * dl + 2);
    const f32x4 oc = {lo.x, lo.y, hi.x, hi.y};
    // an empty chunk carries m = -inf and no o values
    const bool valid = mc != -INFINITY;
    const float mn = valid ? fmaxf(m, mc) : m;
    const float ws = valid ? exp2f(m - mn) : 1.f;
    const float wc = valid ? exp2f(mc - mn) : 0.f;
    l = l * ws + (valid ? lc : 0.f) * wc;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = o[i] * ws + (valid ? oc[i] : 0.f) * wc;
    m = mn;
  }
  *reinterpret_cast<f32x4*>(&s_o[way][4 * dl]) = o;
  if (dl == 0) {
    s_m[way] = m;
    s_l[way] = l;
  }
  __syncthreads();
  if (threadIdx.x >= D) return;
  const int d = threadIdx.x;
  float mt = a.sinks ? a.sinks[h] * kLog2e : -INFINITY;
#pragma unroll
  for (int w = 0; w < kWays; ++w) mt = fmaxf(mt, s_m[w]);
  float lt = (a.sinks && mt != -INFINITY) ? exp2f(a.sinks[h] * kLog2e - mt) : 0.f;
  float ot = 0.f;
#pragma unroll
  for (int w = 0; w < kWays; ++w) {
    if (s_m[w] == -INFINITY) continue;
    const float sw = exp2f(s_m[w] - mt);
    lt += s_l[w] * sw;
    ot += s_o[w][d] * sw;
  }
  const float r = lt > 0.f ? ot / lt : 0.f;
  const int64_t at = static_cast<int64_t>(b) * a.out_stride_b + static_cast<int64_t>(h) * a.out_stride_h + d;
  if (a.out_f32)
    static_cast<float*>(a.out)[at] = r;
  else
    static_cast<__bf16*>(a.out)[at] = static_cast<__bf16>(r);
}

int64_t chunks_for(int64_t max_len) { return max_len <= 0 ? 1 : (max_len + kChunk - 1) / kChunk; }

// Split-K scratch of akv_decode_attention_noalloc: a file-scope device array,
// one per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the
// symbol): it uses the per-device address hipGetSymbolAddress returns.
constexpr int64_t kScratchBytes = 32ll << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up once per device with that
// device current.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return fail(AKV_EHIP, "akv_decode_attention_noalloc: hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(AKV_EINVAL, "akv_decode_attention_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return fail(AKV_EHIP, "akv_decode_attention_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(err));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return AKV_OK;
}

}  // namespace
}  // namespace akv

extern "C" int64_t akv_decode_attention_workspace_bytes(int32_t n_requests, int32_t kv_heads,
                                                         int32_t head_dim, int64_t max_len) {
  using namespace akv;
  if (n_requests < 0 || kv_heads <= 0 || head_dim <= 0 || max_len < 0) return -1;
  return static_cast<int64_t>(n_requests) * kv_heads * chunks_for(max_len) * 16 * (head_dim + 2) * 4;
}

extern "C" int akv_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_buffer,
                                    const void* v_buffer, int64_t k_stride_slot, int64_t k_stride_head,
                                    int64_t v_stride_slot, int64_t v_stride_head, int32_t n_requests,
                                    int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                    const int32_t* kv_indptr, const int32_t* kv_indices, const float* sinks,
                                    float scale, void* out, int32_t out_dtype, int64_t out_stride_b,
                                    int64_t out_stride_h, int64_t max_len, void* workspace,
                                    int64_t workspace_bytes, const int32_t* status, void* stream) {
  using namespace akv;
  if (n_requests < 0 || max_len < 0) return fail(AKV_EINVAL, "akv_decode_attention: negative size");
  if (n_requests == 0) return AKV_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(AKV_EINVAL, "akv_decode_attention: head_dim %d (supported: 64, 128)", head_dim);
  if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0 || q_heads / kv_heads > 16)
    return fail(AKV_EINVAL, "akv_decode_attention: %d q heads over %d KV heads (group <= 16)", q_heads,
                kv_heads);
  if (out_dtype != AKV_BF16 && out_dtype != AKV_F32)
    return fail(AKV_EINVAL, "akv_decode_attention: output must be bf16 or f32");
  if (!q || !k_buffer || !v_buffer || !kv_indptr || !kv_indices || !out || !workspace)
    return fail(AKV_EINVAL, "akv_decode_attention: null device pointer");
  if ((k_stride_slot | k_stride_head | v_stride_slot | v_stride_head) % 8 != 0 ||
      ((reinterpret_cast<uintptr_t>(k_buffer) | reinterpret_cast<uintptr_t>(v_buffer)) & 15) != 0)
    return fail(AKV_EINVAL, "akv_decode_attention: K/V rows must be 16-byte aligned");
  if (n_requests > 65535 || kv_heads > 65535)
    return fail(AKV_EINVAL, "akv_decode_attention: batch too large");
  const int64_t need = akv_decode_attention_workspace_bytes(n_requests, kv_heads, head_dim, max_len);
  if (workspace_bytes < need)
    return fail(AKV_EINVAL, "akv_decode_attention: workspace holds %lld bytes, needs %lld",
                static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  AttnArgs a{};
  a.q = static_cast<const __bf16*>(q);
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k = static_cast<const __bf16*>(k_buffer);
  a.v = static_cast<const __bf16*>(v_buffer);
  a.k_stride_slot = k_stride_slot;
  a.k_stride_head = k_stride_head;
  a.v_stride_slot = v_stride_slot;
  a.v_stride_head = v_stride_head;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.sinks = sinks;
  a.gate = status;
  a.scale_log2 = scale * kLog2e;
  a.out = out;
  a.out_f32 = out_dtype == AKV_F32;
  a.out_stride_b = out_stride_b;
  a.out_stride_h = out_stride_h;
  a.n_requests = n_requests;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.group = q_heads / kv_heads;
  a.chunks = static_cast<int32_t>(chunks_for(max_len));
  a.partial = static_cast<float*>(workspace);
  hipStream_t st = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(a.chunks), static_cast<unsigned>(kv_heads),
                  static_cast<unsigned>(n_requests));
  const dim3 block(64);
  if (head_dim == 64) {
    hipLaunchKernelGGL(decode_attention_partial_kernel<64>, grid, block, 0, st, a);
    int rc = check_launch("akv_decode_attention (partial)");
    if (rc || a.chunks == 1) return rc;
    hipLaunchKernelGGL(decode_attention_combine_kernel<64>, dim3(n_requests, q_heads), dim3(kCombineThreads), 0,
                       st, a);
  } else {
    hipLaunchKernelGGL(decode_attention_partial_kernel<128>, grid, block, 0, st, a);
    int rc = check_launch("akv_decode_attention (partial)");
    if (rc || a.chunks == 1) return rc;
    hipLaunchKernelGGL(decode_attention_combine_kernel<128>, dim3(n_requests, q_heads), dim3(kCombineThreads), 0,
                       st, a);
  }
  return check_launch("akv_decode_attention (combine)");
}

extern "C" int64_t akv_decode_attention_noalloc_max_bytes(void) { return akv::kScratchBytes; }

extern "C" int akv_decode_attention_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                            const void* k_buffer, const void* v_buffer, int64_t k_stride_slot,
                                            int64_t k_stride_head, int64_t v_stride_slot, int64_t v_stride_head,
                                            int32_t n_requests, int32_t q_heads, int32_t kv_heads,
                                            int32_t head_dim, const int32_t* kv_indptr, const int32_t* kv_indices,
                                            const float* sinks, float scale, void* out, int32_t out_dtype,
                                            int64_t out_stride_b, int64_t out_stride_h, int64_t max_len,
                                            const int32_t* status, void* stream) {
  using namespace akv;
  const int64_t need = akv_decode_attention_workspace_bytes(n_requests, kv_heads > 0 ? kv_heads : 1,
                                                            head_dim > 0 ? head_dim : 1, max_len);
  if (need > kScratchBytes)
    return fail(AKV_EINVAL,
                "akv_decode_attention_noalloc: the split-K partials need %lld bytes, the static scratch holds "
                "%lld (%d requests x %d KV heads x max_len %lld)",
                static_cast<long long>(need), static_cast<long long>(kScratchBytes), n_requests, kv_heads,
                static_cast<long long>(max_len));
  if (n_requests <= 0) return akv_decode_attention(q, q_stride_b, q_stride_h, k_buffer, v_buffer, k_stride_slot,
                                                   k_stride_head, v_stride_slot, v_stride_head, n_requests,
                                                   q_heads, kv_heads, head_dim, kv_indptr, kv_indices, sinks,
                                                   scale, out, out_dtype, out_stride_b, out_stride_h, max_len,
                                                   nullptr, 0, status, stream);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return akv_decode_attention(q, q_stride_b, q_stride_h, k_buffer, v_buffer, k_stride_slot, k_stride_head,
                              v_stride_slot, v_stride_head, n_requests, q_heads, kv_heads, head_dim, kv_indptr,
                              kv_indices, sinks, scale, out, out_dtype, out_stride_b, out_stride_h, max_len, ws,
                              kScratchBytes, status, stream);
}
