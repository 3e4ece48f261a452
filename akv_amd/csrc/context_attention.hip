// Prefill context attention over occurrence metadata (gfx950, MFMA).
//
// The extend attention the context system launches once per layer
// (akv/system/sglang/srt/layers/attention/context_backend.py:180-251 and the
// position-aware SWA mask of akv/system/sglang.patch:106-237).  For segment s
// the queries are q[qo_indptr[s] .. qo_indptr[s+1]) and the keys are
//   prefix: pool rows kv_indices[kv_indptr[s] .. kv_indptr[s+1]), all visible;
//   extend: the segment's own K/V rows (k_ext/v_ext aligned with q), causal
//           by index (key j visible to query i when j <= i);
// and, with a sliding window W >= 0, a key at position p_k is visible to a
// query at position p_q only when p_q <= p_k + W.  Positions come from
// q_positions (aligned with q) and kv_positions (aligned with kv_indices);
// without them a query's position is prefix_length + i and a prefix key's
// is its index (the native contiguous case).  Sinks add e^{sink} to the
// softmax denominator.  Within a segment positions ascend (the keys of a
// context window are ordered), which lets a workgroup start the prefix and
// extend loops at the first key inside the window.
//
// Workgroup = (block of 128 / G query tokens, KV head g, segment), with the
// G q heads of the group packed as rows: row r = token * G + head, 128 rows,
// 4 waves x 32 rows.  Per 64-key tile (K and V^T staged in LDS, double
// buffered, the next tile's global loads in flight during this tile's math):
//   S^T[64 keys x 32 rows] = K . Q^T          v_mfma_f32_16x16x32_bf16
//   online softmax per row (column of S^T) in the exp2 domain
//   O^T[D x 32 rows] += V^T . P^T             v_mfma_f32_16x16x32_bf16
// P^T leaves the first MFMA in the B-operand layout of the second (any
// consistent split of the 32-long k axis over lanes gives the same product:
// lane l uses keys 4(l/16)+i of two 16-key subtiles).
//
// MFMA 16x16x32 bf16 lane layout (verified on gfx950): lane l supplies
// A[l%16][k(l,i)], B[k(l,i)][l%16] for i < 8 and holds D[4(l/16)+i][l%16].
#include <cmath>

#include "common.h"

namespace akv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) u32x4 global_u32x4;

constexpr int kRows = 128;  // (token, head) rows per workgroup
constexpr int kThreads = 256;
constexpr int kKeys = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

struct CtxArgs {
  const __bf16* q;
  int64_t q_st, q_sh;
  const __bf16* k_ext;
  const __bf16* v_ext;
  int64_t ke_st, ke_sh, ve_st, ve_sh;
  const __bf16* k_pool;
  const __bf16* v_pool;
  int64_t kp_ss, kp_sh, vp_ss, vp_sh;
  const void* qo_indptr;
  const void* kv_indptr;
  const void* kv_indices;
  const void* q_pos;
  const void* kv_pos;
  int32_t indptr_i64, indices_i64, pos_i64;
  int32_t window;
  const float* sinks;
  float scale_log2;
  void* out;
  int32_t out_f32;
  int64_t o_st, o_sh;
  int32_t kv_heads, group, tokens_per_block;
};

__device__ __forceinline__ u32x4 load16(const __bf16* p) {
  return *((const global_u32x4*)p);
}

template <int D>
struct Smem {
  __bf16 k[2][kKeys][D + 8];       // key-major K tile, rows padded by 16 B
  __bf16 vt[2][D][kKeys + 4];      // dim-major V tile, rows padded by 8 B
  int64_t pos[2][kKeys];           // key positions
};

template <int D>
__global__ void __launch_bounds__(kThreads) context_attention_kernel(const CtxArgs a) {
  constexpr int kChunks = D / 8;                          // 16 B chunks per key row
  constexpr int kKLoads = kKeys * kChunks / kThreads;     // K chunks per thread
  constexpr int kVLoads = (kKeys / 2) * kChunks / kThreads;  // V key-pair chunks per thread
  constexpr int kKSteps = D / 32;                         // MFMA k-steps over head dims
  constexpr int kDTiles = D / 16;                         // O^T row tiles
  __shared__ __attribute__((aligned(16))) Smem<D> sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int quad = lane >> 4;
  const int seg = blockIdx.z;
  const int g = blockIdx.y;
  const bool i64 = a.indptr_i64;
  const int64_t qo0 = load_index(a.qo_indptr, i64, seg);
  const int64_t qlen = load_index(a.qo_indptr, i64, seg + 1) - qo0;
  const int G = a.group;
  const int T = a.tokens_per_block;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * T;
  if (t0 >= qlen) return;
  const int64_t kv0 = load_index(a.kv_indptr, i64, seg);
  const int64_t plen = load_index(a.kv_indptr, i64, seg + 1) - kv0;
  const bool have_pos = a.q_pos != nullptr;
  auto qpos_of = [&](int64_t i) -> int64_t {  // position of query i of the segment
    return have_pos ? load_index(a.q_pos, a.pos_i64, qo0 + i) : plen + i;
  };
  auto kpos_of = [&](int64_t j) -> int64_t {  // position of prefix key j
    return have_pos ? load_index(a.kv_pos, a.pos_i64, kv0 + j) : j;
  };

  // key ranges: prefix [p_lo, plen), extend [e_lo, e_hi)
  const int64_t e_hi = qlen < t0 + T ? qlen : t0 + T;
  int64_t p_lo = 0, e_lo = 0;
  if (a.window >= 0) {
    const int64_t first = qpos_of(t0) - a.window;  // keys below this position are out of every row's window
    int64_t lo = 0, hi = plen;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (kpos_of(mid) < first) lo = mid + 1; else hi = mid;
    }
    p_lo = lo;
    lo = 0;
    hi = t0;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (qpos_of(mid) < first) lo = mid + 1; else hi = mid;
    }
    e_lo = lo;
  }
  const int n_pref = static_cast<int>((plen - p_lo + kKeys - 1) / kKeys);
  const int n_tiles = n_pref + static_cast<int>((e_hi - e_lo + kKeys - 1) / kKeys);

  // this lane's rows: row subtile s covers rows wave*32 + 16s + col
  int64_t row_tok[2], row_pos[2];
  bool row_ok[2];
  int row_head[2];
  bf16x8 qop[2][kKSteps];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int r = wave * 32 + 16 * s + col;
    const int tl = r / G;
    row_head[s] = g * G + (r - tl * G);
    row_tok[s] = t0 + tl;
    row_ok[s] = tl < T && row_tok[s] < qlen;
    row_pos[s] = row_ok[s] ? qpos_of(row_tok[s]) : 0;
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (row_ok[s])
        w = load16(a.q + (qo0 + row_tok[s]) * a.q_st + row_head[s] * a.q_sh + 32 * ks + 8 * quad);
      qop[s][ks] = __builtin_bit_cast(bf16x8, w);
    }
  }

  // tile staging: global -> registers -> LDS
  u32x4 kreg[kKLoads];
  u32x4 vreg[kVLoads][2];
  int64_t preg = 0;
  auto key_src = [&](int it, int key, bool& ok, const __bf16*& kr, const __bf16*& vr) {
    if (it < n_pref) {
      const int64_t j = p_lo + static_cast<int64_t>(it) * kKeys + key;
      ok = j < plen;
      if (ok) {
        const int64_t slot = load_index(a.kv_indices, a.indices_i64, kv0 + j);
        kr = a.k_pool + slot * a.kp_ss + g * a.kp_sh;
        vr = a.v_pool + slot * a.vp_ss + g * a.vp_sh;
      }
    } else {
      const int64_t j = e_lo + static_cast<int64_t>(it - n_pref) * kKeys + key;
      ok = j < e_hi;
      if (ok) {
        kr = a.k_ext + (qo0 + j) * a.ke_st + g * a.ke_sh;
        vr = a.v_ext + (qo0 + j) * a.ve_st + g * a.ve_sh;
      }
    }
  };
  auto stage = [&](int it) {
#pragma unroll
    for (int u = 0; u < kKLoads; ++u) {
      const int c = tid + kThreads * u;
      const int key = c / kChunks;
      const int cc = c - key * kChunks;
      bool ok;
      const __bf16 *kr = nullptr, *vr = nullptr;
      key_src(it, key, ok, kr, vr);
      kreg[u] = ok ? load16(kr + 8 * cc) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kVLoads; ++u) {
      const int c = tid + kThreads * u;
      const int pair = c / kChunks;
      const int cc = c - pair * kChunks;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        bool ok;
        const __bf16 *kr = nullptr, *vr = nullptr;
        key_src(it, 2 * pair + e, ok, kr, vr);
        vreg[u][e] = ok ? load16(vr + 8 * cc) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    if (tid < kKeys) {
      if (it < n_pref) {
        const int64_t j = p_lo + static_cast<int64_t>(it) * kKeys + tid;
        preg = j < plen ? kpos_of(j) : 0;
      } else {
        const int64_t j = e_lo + static_cast<int64_t>(it - n_pref) * kKeys + tid;
        preg = j < e_hi ? qpos_of(j) : 0;
      }
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kKLoads; ++u) {
      const int c = tid + kThreads * u;
      const int key = c / kChunks;
      const int cc = c - key * kChunks;
      *reinterpret_cast<u32x4*>(&sm.k[buf][key][8 * cc]) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < kVLoads; ++u) {
      const int c = tid + kThreads * u;
      const int pair = c / kChunks;
      const int cc = c - pair * kChunks;
      // 8 dims x 2 keys -> 8 words of vt[dim][2 pair .. 2 pair + 1]
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = vreg[u][0][w];
        const uint32_t hi = vreg[u][1][w];
        *reinterpret_cast<uint32_t*>(&sm.vt[buf][8 * cc + 2 * w][2 * pair]) = (lo & 0xffffu) | (hi << 16);
        *reinterpret_cast<uint32_t*>(&sm.vt[buf][8 * cc + 2 * w + 1][2 * pair]) = (lo >> 16) | (hi & 0xffff0000u);
      }
    }
    if (tid < kKeys) sm.pos[buf][tid] = preg;
  };

  f32x4 oacc[kDTiles][2];
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) oacc[dt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};

  stage(0);
  commit(0);
  __syncthreads();
  for (int it = 0; it < n_tiles; ++it) {
    const int buf = it & 1;
    if (it + 1 < n_tiles) stage(it + 1);
    const bool ext = it >= n_pref;
    const int64_t base = ext ? e_lo + static_cast<int64_t>(it - n_pref) * kKeys
                             : p_lo + static_cast<int64_t>(it) * kKeys;
    const int64_t limit = ext ? e_hi : plen;

    // S^T = K . Q^T
    f32x4 sacc[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int s = 0; s < 2; ++s) sacc[kt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kKSteps; ++ks) {
        const bf16x8 kop =
            __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&sm.k[buf][16 * kt + col][32 * ks + 8 * quad]));
#pragma unroll
        for (int s = 0; s < 2; ++s)
          sacc[kt][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[s][ks], sacc[kt][s], 0, 0, 0);
      }
    }

    // mask, online softmax (rows are columns of S^T: lanes col, col+16, col+32, col+48)
    bf16x8 pop[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float sc[4][4];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = 16 * kt + 4 * quad + i;
          const int64_t j = base + key;
          bool vis = row_ok[s] && j < limit;
          if (ext) vis = vis && j <= row_tok[s];
          if (a.window >= 0) vis = vis && row_pos[s] <= sm.pos[buf][key] + a.window;
          sc[kt][i] = vis ? sacc[kt][s][i] * a.scale_log2 : -INFINITY;
          mx = fmaxf(mx, sc[kt][i]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run[s], mx);
      const bool live = m_new != -INFINITY;
      const float alpha = live ? exp2f(m_run[s] - m_new) : 1.f;
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = live ? exp2f(sc[kt][i] - m_new) : 0.f;
          sc[kt][i] = p;
          psum += p;
        }
      l_run[s] = l_run[s] * alpha + psum;
      m_run[s] = m_new;
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) oacc[dt][s] *= alpha;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pop[s][kk][i] = static_cast<__bf16>(sc[2 * kk][i]);
          pop[s][kk][4 + i] = static_cast<__bf16>(sc[2 * kk + 1][i]);
        }
    }

    // O^T += V^T . P^T
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(&sm.vt[buf][16 * dt + col][32 * kk + 4 * quad]);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(&sm.vt[buf][16 * dt + col][32 * kk + 16 + 4 * quad]);
        const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
        const bf16x8 vop = __builtin_bit_cast(bf16x8, w);
#pragma unroll
        for (int s = 0; s < 2; ++s)
          oacc[dt][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[s][kk], oacc[dt][s], 0, 0, 0);
      }

    if (it + 1 < n_tiles) commit(buf ^ 1);
    __syncthreads();
  }

  // normalise (row sums over the 4 lanes of a column) with the sink; store
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float l = l_run[s];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    float scale = 1.f;
    if (a.sinks) {
      const float sink = a.sinks[row_head[s]] * kLog2e;
      const float m_f = fmaxf(m_run[s], sink);
      scale = m_run[s] == -INFINITY ? 0.f : exp2f(m_run[s] - m_f);
      l = l * scale + exp2f(sink - m_f);
    }
    const float inv = l > 0.f ? scale / l : 0.f;
    if (!row_ok[s]) continue;
    const int64_t at = (qo0 + row_tok[s]) * a.o_st + row_head[s] * a.o_sh + 4 * quad;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) {
      const f32x4 o = oacc[dt][s] * inv;
      if (a.out_f32) {
        *reinterpret_cast<f32x4*>(static_cast<float*>(a.out) + at + 16 * dt) = o;
      } else {
        bf16x4 ob;
#pragma unroll
        for (int i = 0; i < 4; ++i) ob[i] = static_cast<__bf16>(o[i]);
        *reinterpret_cast<bf16x4*>(static_cast<__bf16*>(a.out) + at + 16 * dt) = ob;
      }
    }
  }
}

}  // namespace
}  // namespace akv

extern "C" int akv_context_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_ext,
                                     const void* v_ext, int64_t k_ext_stride_t, int64_t k_ext_stride_h,
                                     int64_t v_ext_stride_t, int64_t v_ext_stride_h, const void* k_buffer,
                                     const void* v_buffer, int64_t k_stride_slot, int64_t k_stride_head,
                                     int64_t v_stride_slot, int64_t v_stride_head, int32_t n_segments,
                                     int32_t q_heads, int32_t kv_heads, int32_t head_dim, const void* qo_indptr,
                                     const void* kv_indptr, int32_t indptr_dtype, const void* kv_indices,
                                     int32_t indices_dtype, const void* q_positions, const void* kv_positions,
                                     int32_t positions_dtype, int32_t sliding_window, const float* sinks,
                                     float scale, void* out, int32_t out_dtype, int64_t out_stride_t,
                                     int64_t out_stride_h, int64_t max_query_len, void* stream) {
  using namespace akv;
  if (n_segments < 0 || max_query_len < 0) return fail(AKV_EINVAL, "akv_context_attention: negative size");
  if (n_segments == 0 || max_query_len == 0) return AKV_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(AKV_EINVAL, "akv_context_attention: head_dim %d (supported: 64, 128)", head_dim);
  if (kv_heads <= 0 || q_heads % kv_heads != 0 || kRows % (q_heads / kv_heads) != 0)
    return fail(AKV_EINVAL, "akv_context_attention: %d q heads over %d KV heads (group must divide %d)",
                q_heads, kv_heads, kRows);
  if (!valid_index_dtype(indptr_dtype) || !valid_index_dtype(indices_dtype) ||
      !valid_index_dtype(positions_dtype))
    return fail(AKV_EINVAL, "akv_context_attention: index vectors must be int32 or int64");
  if (out_dtype != AKV_BF16 && out_dtype != AKV_F32)
    return fail(AKV_EINVAL, "akv_context_attention: output must be bf16 or f32");
  if (!q || !k_ext || !v_ext || !out || !qo_indptr || !kv_indptr)
    return fail(AKV_EINVAL, "akv_context_attention: null device pointer");
  if ((q_positions == nullptr) != (kv_positions == nullptr))
    return fail(AKV_EINVAL, "akv_context_attention: needs both query and KV positions or neither");
  const int64_t strides[] = {q_stride_t,    q_stride_h,    k_ext_stride_t, k_ext_stride_h, v_ext_stride_t,
                             v_ext_stride_h, k_stride_slot, k_stride_head,  v_stride_slot,  v_stride_head,
                             out_stride_t,  out_stride_h};
  for (int64_t s : strides)
    if (s % 8 != 0) return fail(AKV_EINVAL, "akv_context_attention: row strides must be multiples of 8 elements");
  const uintptr_t bases = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_ext) |
                          reinterpret_cast<uintptr_t>(v_ext) | reinterpret_cast<uintptr_t>(k_buffer) |
                          reinterpret_cast<uintptr_t>(v_buffer) | reinterpret_cast<uintptr_t>(out);
  if (bases & 15) return fail(AKV_EINVAL, "akv_context_attention: tensors must be 16-byte aligned");
  if (n_segments > 65535 || kv_heads > 65535)
    return fail(AKV_EINVAL, "akv_context_attention: batch too large");
  CtxArgs a{};
  a.q = static_cast<const __bf16*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.k_ext = static_cast<const __bf16*>(k_ext);
  a.v_ext = static_cast<const __bf16*>(v_ext);
  a.ke_st = k_ext_stride_t;
  a.ke_sh = k_ext_stride_h;
  a.ve_st = v_ext_stride_t;
  a.ve_sh = v_ext_stride_h;
  a.k_pool = static_cast<const __bf16*>(k_buffer);
  a.v_pool = static_cast<const __bf16*>(v_buffer);
  a.kp_ss = k_stride_slot;
  a.kp_sh = k_stride_head;
  a.vp_ss = v_stride_slot;
  a.vp_sh = v_stride_head;
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.q_pos = q_positions;
  a.kv_pos = kv_positions;
  a.indptr_i64 = indptr_dtype == AKV_I64;
  a.indices_i64 = indices_dtype == AKV_I64;
  a.pos_i64 = positions_dtype == AKV_I64;
  a.window = sliding_window < 0 ? -1 : sliding_window;
  a.sinks = sinks;
  a.scale_log2 = scale * kLog2e;
  a.out = out;
  a.out_f32 = out_dtype == AKV_F32;
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.kv_heads = kv_heads;
  a.group = q_heads / kv_heads;
  a.tokens_per_block = kRows / a.group;
  const int64_t blocks = (max_query_len + a.tokens_per_block - 1) / a.tokens_per_block;
  if (blocks > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_context_attention: queries too long");
  const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(kv_heads), static_cast<unsigned>(n_segments));
  hipStream_t st = as_stream(stream);
  if (head_dim == 64)
    hipLaunchKernelGGL(context_attention_kernel<64>, grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(context_attention_kernel<128>, grid, dim3(kThreads), 0, st, a);
  return check_launch("akv_context_attention");
}
