// Fused all-layer Reposition for gfx950: K re-rotation + K tail / V move.
//
// Semantics follow _reposition_layers_kernel,
// akv/system/sglang/kernels/ops/attention/context_reposition.py:28-123:
// per (token, layer, head), fp32 inverse rotation by the old position (IEEE
// division by cos^2 + sin^2) followed by the forward rotation by the new
// position, every product and sum rounded on its own (this file is built with
// -ffp-contract=off), round-to-nearest-even store; same position stores the
// source bits; K dims [R, D) and all of V are copied bit for bit.
//
// MI355X design (not the reference's one-program-per-(token, layer, head)
// grid): one workgroup per moved token walks every layer of the group, so the
// token's slots, positions and its cos/sin rows are read once and kept in
// registers (and cos^2 + sin^2 computed once) instead of once per
// (layer, head).  Each lane owns one "rotary unit" of a head: for NeoX style
// the 16-byte chunk at i and its partner chunk at i + R/2, so both halves of
// every pair sit in the same lane and no cross-lane exchange is needed; for
// GPT-J style one 16-byte chunk of interleaved pairs.  K and V move as 16-byte
// vector accesses; a 64-lane wave covers 1 KiB of contiguous K (and V) per
// instruction for the 8 x 64 bf16 head layout.  Layers whose base address is
// not 16-byte aligned take an element-wise path inside the same kernel; other
// shapes go to a generic element-per-thread kernel.
#include <cstdlib>

#include "common.h"

namespace akv {
namespace {

struct RepositionArgs {
  const uint64_t* k_ptrs;
  const uint64_t* v_ptrs;
  const int32_t* src;
  const int32_t* dst;
  const int32_t* pairs;
  const void* cos_sin;
  int64_t k_stride_slot, k_stride_head, v_stride_slot, v_stride_head;
  int64_t pair_stride, rope_stride;
  int32_t n_layers, n_heads, head_dim, rotary_dim;
  int32_t skip_unmapped;
  int32_t is_neox;
  int32_t units_per_head;  // rotary units per head
  int32_t lanes_per_row;   // n_heads * units_per_head
  int32_t rows_per_block;  // layers processed side by side by one token
  int32_t tokens_per_block;
  int64_t n_tokens;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4 make_u32x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 r = {a, b, c, d};
  return r;
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static constexpr int kVec = 4;
};
template <>
struct Elem<_Float16> {
  static constexpr int kVec = 8;
};
template <>
struct Elem<__bf16> {
  static constexpr int kVec = 8;
};

__device__ __forceinline__ float to_float(float x) { return x; }
__device__ __forceinline__ float to_float(_Float16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_float(__bf16 x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_float(float x);
template <>
__device__ __forceinline__ float from_float<float>(float x) { return x; }
template <>
__device__ __forceinline__ _Float16 from_float<_Float16>(float x) {
  return static_cast<_Float16>(x);
}
template <>
__device__ __forceinline__ __bf16 from_float<__bf16>(float x) {
  return static_cast<__bf16>(x);
}

// 16 bytes of storage <-> fp32 values.
template <typename T>
__device__ __forceinline__ void unpack(const u32x4 u, float (&f)[Elem<T>::kVec]);

template <>
__device__ __forceinline__ void unpack<__bf16>(const u32x4 u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void unpack<_Float16>(const u32x4 u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f16x2_t h = __builtin_bit_cast(f16x2_t, w[k]);
    f[2 * k] = static_cast<float>(h.x);
    f[2 * k + 1] = static_cast<float>(h.y);
  }
}

template <>
__device__ __forceinline__ void unpack<float>(const u32x4 u, float (&f)[4]) {
  f[0] = __uint_as_float(u.x);
  f[1] = __uint_as_float(u.y);
  f[2] = __uint_as_float(u.z);
  f[3] = __uint_as_float(u.w);
}

template <typename T>
__device__ __forceinline__ u32x4 pack(const float (&f)[Elem<T>::kVec]);

template <>
__device__ __forceinline__ u32x4 pack<__bf16>(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x2_t v = {f[2 * k], f[2 * k + 1]};
    w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  }
  return make_u32x4(w[0], w[1], w[2], w[3]);
}

template <>
__device__ __forceinline__ u32x4 pack<_Float16>(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x2_t v = {f[2 * k], f[2 * k + 1]};
    w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  }
  return make_u32x4(w[0], w[1], w[2], w[3]);
}

template <>
__device__ __forceinline__ u32x4 pack<float>(const float (&f)[4]) {
  return make_u32x4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                    __float_as_uint(f[3]));
}

// KV rows live in global memory; the layer pointers arrive as plain 64-bit
// addresses, so name the address space to get global_* instead of flat_*
// instructions.
typedef __attribute__((address_space(1))) u32x4 global_u32x4;

// 16-byte load/store; `aligned` is wave-uniform.  Plain (temporal) accesses:
// on MI355X they measured faster than the nontemporal forms for this
// scattered 1 KiB-row pattern (AKV_REPOSITION_NT selects the latter).
template <typename T>
__device__ __forceinline__ u32x4 load16(const T* p, bool aligned) {
#ifdef AKV_REPOSITION_NT
  if (aligned) return __builtin_nontemporal_load((const global_u32x4*)(p));
#else
  if (aligned) return *((const global_u32x4*)(p));
#endif
  union {
    u32x4 u;
    T e[Elem<T>::kVec];
  } r;
#pragma unroll
  for (int k = 0; k < Elem<T>::kVec; ++k) r.e[k] = p[k];
  return r.u;
}

template <typename T>
__device__ __forceinline__ void store16(T* p, u32x4 v, bool aligned) {
  if (aligned) {
#ifdef AKV_REPOSITION_NT
    __builtin_nontemporal_store(v, (global_u32x4*)(p));
#else
    *((global_u32x4*)(p)) = v;
#endif
    return;
  }
  union {
    u32x4 u;
    T e[Elem<T>::kVec];
  } r;
  r.u = v;
#pragma unroll
  for (int k = 0; k < Elem<T>::kVec; ++k) p[k] = r.e[k];
}

// Loads NP consecutive table values as fp32.  The host guarantees that the
// table base, its row stride and every unit offset are multiples of the
// vector size.
template <typename CS, int NP>
__device__ __forceinline__ void load_table(const CS* p, float (&out)[NP]) {
  typedef CS vec_t __attribute__((ext_vector_type(NP)));
  const vec_t v = *reinterpret_cast<const vec_t*>(p);
#pragma unroll
  for (int k = 0; k < NP; ++k) out[k] = to_float(v[k]);
}

// The reference rotation, op for op (context_reposition.py:92-102).
__device__ __forceinline__ void rotate(float x1, float x2, float co, float so, float s,
                                       float cn, float sn, float& y1, float& y2) {
  const float u1 = (x1 * co + x2 * so) / s;
  const float u2 = (x2 * co - x1 * so) / s;
  y1 = u1 * cn - u2 * sn;
  y2 = u2 * cn + u1 * sn;
}

// Registers of one (token, layer) row between its loads and its stores.
struct RowData {
  u32x4 k1, k2;  // rotary unit of K (the partner half for NeoX style)
  u32x4 v[2];    // this lane's first two V units
  uintptr_t kb, vb;
  bool aligned;
};

template <typename T, typename CS, bool NEOX>
struct RowMover {
  static constexpr int VEC = Elem<T>::kVec;
  static constexpr int NP = NEOX ? VEC : VEC / 2;  // rotation pairs per lane
  const RepositionArgs& a;
  int64_t src, dst;
  int h, j, off1, off2, lpr, v_units_head, v_units_row, t_units_head, t_units_row;
  bool same;
  float co[NP], so[NP], cn[NP], sn[NP], s2[NP];

  __device__ __forceinline__ RowData load(int layer) const {
    RowData r;
    r.kb = static_cast<uintptr_t>(a.k_ptrs[layer]);
    r.vb = static_cast<uintptr_t>(a.v_ptrs[layer]);
    // one wave may hold rows of several layers: take the vector path only
    // when every row of the wave is 16-byte aligned (a uniform branch)
    r.aligned = __ballot(((r.kb | r.vb) & 15) != 0) == 0;
    const T* ks = reinterpret_cast<const T*>(r.kb) + src * a.k_stride_slot + h * a.k_stride_head;
    r.k1 = load16(ks + off1, r.aligned);
    r.k2 = NEOX ? load16(ks + off2, r.aligned) : make_u32x4(0, 0, 0, 0);
    const T* vs = reinterpret_cast<const T*>(r.vb) + src * a.v_stride_slot;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int c = j + q * lpr;
      if (c < v_units_row) {
        const int vh = c / v_units_head;
        r.v[q] = load16(vs + vh * a.v_stride_head + (c - vh * v_units_head) * VEC, r.aligned);
      }
    }
    return r;
  }

  __device__ __forceinline__ void finish(const RowData& r) const {
    T* kb = reinterpret_cast<T*>(r.kb);
    T* vb = reinterpret_cast<T*>(r.vb);
    T* kd = kb + dst * a.k_stride_slot + h * a.k_stride_head;
    u32x4 o1 = r.k1, o2 = r.k2;
    if (!same) {
      float x1[VEC], x2[VEC], y1[VEC], y2[VEC];
      unpack<T>(r.k1, x1);
      if (NEOX) {
        unpack<T>(r.k2, x2);
#pragma unroll
        for (int k = 0; k < NP; ++k) rotate(x1[k], x2[k], co[k], so[k], s2[k], cn[k], sn[k], y1[k], y2[k]);
        o1 = pack<T>(y1);
        o2 = pack<T>(y2);
      } else {
#pragma unroll
        for (int k = 0; k < NP; ++k)
          rotate(x1[2 * k], x1[2 * k + 1], co[k], so[k], s2[k], cn[k], sn[k], y1[2 * k], y1[2 * k + 1]);
        o1 = pack<T>(y1);
      }
    }
    store16(kd + off1, o1, r.aligned);
    if (NEOX) store16(kd + off2, o2, r.aligned);
    const T* vs = vb + src * a.v_stride_slot;
    T* vd = vb + dst * a.v_stride_slot;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int c = j + q * lpr;
      if (c < v_units_row) {
        const int vh = c / v_units_head;
        store16(vd + vh * a.v_stride_head + (c - vh * v_units_head) * VEC, r.v[q], r.aligned);
      }
    }
    // V units beyond two per lane (wide heads with few rotary units)
    for (int c = j + 2 * lpr; c < v_units_row; c += lpr) {
      const int vh = c / v_units_head;
      const int ve = (c - vh * v_units_head) * VEC;
      store16(vd + vh * a.v_stride_head + ve, load16(vs + vh * a.v_stride_head + ve, r.aligned), r.aligned);
    }
    // K tail dims [R, D)
    for (int c = j; c < t_units_row; c += lpr) {
      const int th = c / t_units_head;
      const int te = a.rotary_dim + (c - th * t_units_head) * VEC;
      const T* ts = kb + src * a.k_stride_slot + th * a.k_stride_head + te;
      T* td = kb + dst * a.k_stride_slot + th * a.k_stride_head + te;
      store16(td, load16(ts, r.aligned), r.aligned);
    }
  }
};

// Workgroup = tokens_per_block tokens x rows_per_block layer rows side by
// side x lanes_per_row lanes; each lane walks the layers of its token.
template <typename T, typename CS, bool NEOX>
__global__ void __launch_bounds__(1024) reposition_vec_kernel(const RepositionArgs a) {
  using Mover = RowMover<T, CS, NEOX>;
  constexpr int VEC = Mover::VEC;
  constexpr int NP = Mover::NP;
  const int lpr = a.lanes_per_row;
  const int row_threads = lpr * a.rows_per_block;
  const int slot = threadIdx.x / row_threads;
  const int local = threadIdx.x - slot * row_threads;
  const int row_sub = local / lpr;
  const int j = local - row_sub * lpr;
  const int64_t token = static_cast<int64_t>(blockIdx.x) * a.tokens_per_block + slot;
  if (slot >= a.tokens_per_block || token >= a.n_tokens) return;

  Mover mv{a};
  mv.src = a.src[token];
  mv.dst = a.dst[token];
  if (a.skip_unmapped && (mv.src <= 0 || mv.dst <= 0)) return;
  const int32_t* pair = a.pairs + token * a.pair_stride;
  const int64_t old_pos = pair[0];
  const int64_t new_pos = pair[1];
  mv.same = old_pos == new_pos;
  const int half = a.rotary_dim >> 1;
  mv.lpr = lpr;
  mv.j = j;
  mv.h = j / a.units_per_head;
  const int g = j - mv.h * a.units_per_head;
  mv.off1 = g * VEC;
  mv.off2 = NEOX ? half + g * VEC : 0;
  const int i0 = NEOX ? g * VEC : g * (VEC / 2);
  mv.v_units_head = a.head_dim / VEC;
  mv.v_units_row = a.n_heads * mv.v_units_head;
  mv.t_units_head = (a.head_dim - a.rotary_dim) / VEC;
  mv.t_units_row = a.n_heads * mv.t_units_head;
  if (!mv.same) {
    const CS* table = static_cast<const CS*>(a.cos_sin);
    load_table<CS, NP>(table + old_pos * a.rope_stride + i0, mv.co);
    load_table<CS, NP>(table + old_pos * a.rope_stride + half + i0, mv.so);
    load_table<CS, NP>(table + new_pos * a.rope_stride + i0, mv.cn);
    load_table<CS, NP>(table + new_pos * a.rope_stride + half + i0, mv.sn);
#pragma unroll
    for (int k = 0; k < NP; ++k) mv.s2[k] = mv.co[k] * mv.co[k] + mv.so[k] * mv.so[k];
  }

  // Double-buffered over layers: the next row's loads are in flight during
  // this row's arithmetic and stores (measured +2% over load-then-finish).
  if (row_sub < a.n_layers) {
    RowData cur = mv.load(row_sub);
    for (int layer = row_sub; layer < a.n_layers; layer += a.rows_per_block) {
      const int next = layer + a.rows_per_block;
      RowData nxt = cur;
      if (next < a.n_layers) nxt = mv.load(next);
      mv.finish(cur);
      cur = nxt;
    }
  }
}

// Any layout: one thread per (token, layer, head, dim) element.
template <typename T, typename CS>
__global__ void __launch_bounds__(256) reposition_generic_kernel(const RepositionArgs a, int64_t total) {
  const int D = a.head_dim;
  const int H = a.n_heads;
  const int R = a.rotary_dim;
  const int half = R >> 1;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += stride) {
    int64_t rest = idx;
    const int d = static_cast<int>(rest % D);
    rest /= D;
    const int h = static_cast<int>(rest % H);
    rest /= H;
    const int layer = static_cast<int>(rest % a.n_layers);
    const int64_t token = rest / a.n_layers;
    const int64_t src = a.src[token];
    const int64_t dst = a.dst[token];
    if (a.skip_unmapped && (src <= 0 || dst <= 0)) continue;
    T* kb = reinterpret_cast<T*>(a.k_ptrs[layer]);
    T* vb = reinterpret_cast<T*>(a.v_ptrs[layer]);
    const T* ks = kb + src * a.k_stride_slot + h * a.k_stride_head;
    T* kd = kb + dst * a.k_stride_slot + h * a.k_stride_head;
    if (d < half) {
      const int64_t old_pos = a.pairs[token * a.pair_stride];
      const int64_t new_pos = a.pairs[token * a.pair_stride + 1];
      const int e1 = a.is_neox ? d : 2 * d;
      const int e2 = a.is_neox ? d + half : 2 * d + 1;
      const T b1 = ks[e1];
      const T b2 = ks[e2];
      if (old_pos == new_pos) {
        kd[e1] = b1;
        kd[e2] = b2;
      } else {
        const CS* table = static_cast<const CS*>(a.cos_sin);
        const float co = to_float(table[old_pos * a.rope_stride + d]);
        const float so = to_float(table[old_pos * a.rope_stride + half + d]);
        const float cn = to_float(table[new_pos * a.rope_stride + d]);
        const float sn = to_float(table[new_pos * a.rope_stride + half + d]);
        const float s2 = co * co + so * so;
        float y1, y2;
        rotate(to_float(b1), to_float(b2), co, so, s2, cn, sn, y1, y2);
        kd[e1] = from_float<T>(y1);
        kd[e2] = from_float<T>(y2);
      }
    } else if (d >= R) {
      kd[d] = ks[d];
    }
    vb[dst * a.v_stride_slot + h * a.v_stride_head + d] = vb[src * a.v_stride_slot + h * a.v_stride_head + d];
  }
}

int env_int(const char* name) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : 0;
}

// Launch geometry of the vector kernel.  Measured on MI355X for the
// 36-layer x 8-head x 64 bf16 shape: about 192 threads per token (6 layers
// side by side, 6 passes each) beat both one wave per token and one row per
// lane; tokens whose rows fill less than two waves share a workgroup.
// AKV_REPOSITION_ROWS_PER_BLOCK / AKV_REPOSITION_TOKENS_PER_BLOCK override.
void geometry(RepositionArgs& a) {
  const int lpr = a.lanes_per_row;
  const int forced_rows = env_int("AKV_REPOSITION_ROWS_PER_BLOCK");
  int rows = forced_rows > 0 ? forced_rows : 192 / lpr;
  if (rows < 1) rows = 1;
  if (rows > a.n_layers) rows = a.n_layers;
  if (forced_rows <= 0) {
    const int passes = (a.n_layers + rows - 1) / rows;
    rows = (a.n_layers + passes - 1) / passes;  // balance the passes
  }
  while (rows > 1 && rows * lpr > 1024) --rows;
  a.rows_per_block = rows;
  const int forced_tokens = env_int("AKV_REPOSITION_TOKENS_PER_BLOCK");
  int tokens = forced_tokens > 0 ? forced_tokens : 128 / (rows * lpr);
  if (tokens < 1) tokens = 1;
  while (tokens > 1 && tokens * rows * lpr > 1024) --tokens;
  a.tokens_per_block = tokens;
}

template <typename T, typename CS>
int launch_typed(RepositionArgs a, int64_t n_tokens, hipStream_t stream, bool vec_ok) {
  constexpr int VEC = Elem<T>::kVec;
  a.n_tokens = n_tokens;
  if (vec_ok) {
    a.units_per_head = a.is_neox ? a.rotary_dim / (2 * VEC) : a.rotary_dim / VEC;
    a.lanes_per_row = a.n_heads * a.units_per_head;
    geometry(a);
    const int threads = a.lanes_per_row * a.rows_per_block * a.tokens_per_block;
    const dim3 grid(static_cast<unsigned>((n_tokens + a.tokens_per_block - 1) / a.tokens_per_block));
    if (a.is_neox)
      hipLaunchKernelGGL((reposition_vec_kernel<T, CS, true>), grid, dim3(threads), 0, stream, a);
    else
      hipLaunchKernelGGL((reposition_vec_kernel<T, CS, false>), grid, dim3(threads), 0, stream, a);
    return check_launch("akv_reposition_kv_layers");
  }
  const int64_t total = n_tokens * a.n_layers * a.n_heads * a.head_dim;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((reposition_generic_kernel<T, CS>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                     0, stream, a, total);
  return check_launch("akv_reposition_kv_layers");
}

template <typename T>
int launch_cs(RepositionArgs a, int64_t n_tokens, int32_t cs_dtype, hipStream_t st, bool vec_ok) {
  switch (cs_dtype) {
    case AKV_F32:
      return launch_typed<T, float>(a, n_tokens, st, vec_ok);
    case AKV_F16:
      return launch_typed<T, _Float16>(a, n_tokens, st, vec_ok);
    case AKV_BF16:
      return launch_typed<T, __bf16>(a, n_tokens, st, vec_ok);
  }
  return fail(AKV_EINVAL, "akv_reposition_kv_layers: unsupported cos_sin dtype %d", cs_dtype);
}

int dtype_bytes(int32_t d) { return d == AKV_F32 ? 4 : 2; }

}  // namespace
}  // namespace akv

extern "C" int akv_reposition_kv_layers(const uint64_t* k_ptrs, const uint64_t* v_ptrs,
                                        int32_t n_layers, int32_t kv_dtype, int32_t n_heads,
                                        int32_t head_dim, int32_t rotary_dim, int64_t k_stride_slot,
                                        int64_t k_stride_head, int64_t v_stride_slot,
                                        int64_t v_stride_head, const int32_t* src,
                                        const int32_t* dst, const int32_t* pairs,
                                        int64_t pair_stride, int64_t n_tokens, const void* cos_sin,
                                        int32_t cos_sin_dtype, int64_t rope_stride, int32_t is_neox,
                                        int32_t skip_unmapped, void* stream) {
  using namespace akv;
  if (kv_dtype != AKV_F32 && kv_dtype != AKV_F16 && kv_dtype != AKV_BF16)
    return fail(AKV_EINVAL, "akv_reposition_kv_layers: unsupported KV dtype %d", kv_dtype);
  if (cos_sin_dtype != AKV_F32 && cos_sin_dtype != AKV_F16 && cos_sin_dtype != AKV_BF16)
    return fail(AKV_EINVAL, "akv_reposition_kv_layers: unsupported cos_sin dtype %d", cos_sin_dtype);
  if (n_layers < 0 || n_tokens < 0 || n_heads <= 0 || head_dim <= 0)
    return fail(AKV_EINVAL, "akv_reposition_kv_layers: invalid shape (layers %d, tokens %lld, heads %d, head_dim %d)",
                n_layers, static_cast<long long>(n_tokens), n_heads, head_dim);
  if (rotary_dim <= 0 || rotary_dim > head_dim || (rotary_dim & 1))
    return fail(AKV_EINVAL, "akv_reposition_kv_layers: rotary_dim %d must be even and in (0, head_dim]",
                rotary_dim);
  if (n_tokens == 0 || n_layers == 0) return AKV_OK;
  if (!k_ptrs || !v_ptrs || !src || !dst || !pairs || !cos_sin)
    return fail(AKV_EINVAL, "akv_reposition_kv_layers: null device pointer");
  if (n_tokens > 0x7fffffffLL)
    return fail(AKV_EINVAL, "akv_reposition_kv_layers: %lld tokens exceed one launch",
                static_cast<long long>(n_tokens));
  if (pair_stride < 0 || rope_stride < 0)
    return fail(AKV_EINVAL, "akv_reposition_kv_layers: negative pair or rope stride");

  RepositionArgs a{};
  a.k_ptrs = k_ptrs;
  a.v_ptrs = v_ptrs;
  a.src = src;
  a.dst = dst;
  a.pairs = pairs;
  a.cos_sin = cos_sin;
  a.k_stride_slot = k_stride_slot;
  a.k_stride_head = k_stride_head;
  a.v_stride_slot = v_stride_slot;
  a.v_stride_head = v_stride_head;
  a.pair_stride = pair_stride;
  a.rope_stride = rope_stride;
  a.n_layers = n_layers;
  a.n_heads = n_heads;
  a.head_dim = head_dim;
  a.rotary_dim = rotary_dim;
  a.skip_unmapped = skip_unmapped ? 1 : 0;
  a.is_neox = is_neox ? 1 : 0;

  // The vector kernel needs 16-byte units that never straddle a head or the
  // rotary boundary, and a table whose per-lane slices are vector aligned.
  const int vec = 16 / dtype_bytes(kv_dtype);
  const int np = is_neox ? vec : vec / 2;
  const int64_t cs_align = static_cast<int64_t>(np) * dtype_bytes(cos_sin_dtype);
  bool vec_ok = head_dim % vec == 0 && k_stride_slot % vec == 0 && k_stride_head % vec == 0 &&
                v_stride_slot % vec == 0 && v_stride_head % vec == 0 &&
                (is_neox ? rotary_dim % (2 * vec) == 0 : rotary_dim % vec == 0) &&
                (reinterpret_cast<uintptr_t>(cos_sin) % cs_align) == 0 && rope_stride % np == 0 &&
                ((rotary_dim / 2) % np) == 0;
  if (vec_ok) {
    const int units = is_neox ? rotary_dim / (2 * vec) : rotary_dim / vec;
    if (static_cast<int64_t>(n_heads) * units > 1024) vec_ok = false;
  }
  hipStream_t st = as_stream(stream);
  switch (kv_dtype) {
    case AKV_F32:
      return launch_cs<float>(a, n_tokens, cos_sin_dtype, st, vec_ok);
    case AKV_F16:
      return launch_cs<_Float16>(a, n_tokens, cos_sin_dtype, st, vec_ok);
    default:
      return launch_cs<__bf16>(a, n_tokens, cos_sin_dtype, st, vec_ok);
  }
}
