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
// grid): a workgroup moves the rows of about 256 threads' worth of
// consecutive tokens (8 tokens of the 8 x 64 head layout) in one layer, with
// the tokens' cos/sin rows (and cos^2 + sin^2) staged once in LDS for every
// head.  Workgroups sweep token blocks fastest, then layers, in one sweep or
// in token chunks (see the launch geometry below); token blocks come in
// multiples of 8 so that a block meets the same XCD in every layer.  Each
// lane owns one "rotary unit" of a head: for NeoX style
// the 16-byte chunk at i and its partner chunk at i + R/2, so both halves of
// every pair sit in the same lane and no cross-lane exchange is needed; for
// GPT-J style one 16-byte chunk of interleaved pairs.  K and V move as 16-byte
// vector accesses; a 64-lane wave covers 1 KiB of contiguous K (and V) per
// instruction for the 8 x 64 bf16 head layout.  Layers whose base address is
// not 16-byte aligned take an element-wise path inside the same kernel; other
// shapes go to a generic element-per-thread kernel.
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
  const int32_t* gate;  // compaction status word, or nullptr
  int64_t k_stride_slot, k_stride_head, v_stride_slot, v_stride_head;
  int64_t pair_stride, rope_stride;
  int32_t n_layers, n_heads, head_dim, rotary_dim;
  int32_t skip_unmapped;
  int32_t is_neox;
  int32_t units_per_head;    // rotary units per head
  int32_t lanes_per_row;     // n_heads * units_per_head
  int32_t tokens_per_block;  // consecutive tokens side by side in a workgroup
  int32_t layers_per_block;  // layers a workgroup walks, one row per token at a time
  int32_t layer_groups;      // ceil(n_layers / layers_per_block)
  int32_t token_blocks;      // token blocks, rounded up to a multiple of 8
  int32_t chunk_blocks;      // token blocks per chunk (a multiple of 8)
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

// Elements e and e + 1 (e even) of a 16-byte unit held as four 32-bit words,
// to fp32 and back.  For 16-bit types the pair is one word; for fp32 two.
template <typename T>
__device__ __forceinline__ void unpack_two(const uint32_t (&w)[4], int e, float* f);
template <>
__device__ __forceinline__ void unpack_two<__bf16>(const uint32_t (&w)[4], int e, float* f) {
  const uint32_t x = w[e >> 1];
  f[0] = __uint_as_float(x << 16);
  f[1] = __uint_as_float(x & 0xffff0000u);
}
template <>
__device__ __forceinline__ void unpack_two<_Float16>(const uint32_t (&w)[4], int e, float* f) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, w[e >> 1]);
  f[0] = static_cast<float>(h.x);
  f[1] = static_cast<float>(h.y);
}
template <>
__device__ __forceinline__ void unpack_two<float>(const uint32_t (&w)[4], int e, float* f) {
  f[0] = __uint_as_float(w[e]);
  f[1] = __uint_as_float(w[e + 1]);
}

template <typename T>
__device__ __forceinline__ void pack_two(const float* f, int e, uint32_t (&w)[4]);
template <>
__device__ __forceinline__ void pack_two<__bf16>(const float* f, int e, uint32_t (&w)[4]) {
  const f32x2_t v = {f[0], f[1]};
  w[e >> 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
template <>
__device__ __forceinline__ void pack_two<_Float16>(const float* f, int e, uint32_t (&w)[4]) {
  const f32x2_t v = {f[0], f[1]};
  w[e >> 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}
template <>
__device__ __forceinline__ void pack_two<float>(const float* f, int e, uint32_t (&w)[4]) {
  w[e] = __float_as_uint(f[0]);
  w[e + 1] = __float_as_uint(f[1]);
}

// KV rows live in global memory; the layer pointers arrive as plain 64-bit
// addresses, so name the address space to get global_* instead of flat_*
// instructions.
typedef __attribute__((address_space(1))) u32x4 global_u32x4;

// 16-byte load/store; ALIGNED is decided once per workgroup.  Loads are
// plain (temporal); stores are nontemporal: the kernel never reads a
// destination row back, and streaming the writes past the caches measured
// faster on MI355X (ascending slots +4-5%, random +0.4-2.3%, page-16
// copy-on-write +0.8%), where nontemporal loads as well were far slower.
template <bool ALIGNED, typename T>
__device__ __forceinline__ u32x4 load16(const T* p) {
  if (ALIGNED) return *((const global_u32x4*)(p));
  union {
    u32x4 u;
    T e[Elem<T>::kVec];
  } r;
#pragma unroll
  for (int k = 0; k < Elem<T>::kVec; ++k) r.e[k] = p[k];
  return r.u;
}

template <bool ALIGNED, typename T>
__device__ __forceinline__ void store16(T* p, u32x4 v) {
  if (ALIGNED) {
    __builtin_nontemporal_store(v, (global_u32x4*)(p));
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

// Floats between the coefficient arrays of one token in LDS: `half`
// rounded up to 8 so every array starts 32-byte aligned.
__host__ __device__ __forceinline__ int coef_stride(int half) { return (half + 7) & ~7; }

// Two coefficients from LDS.
__device__ __forceinline__ float2 lds2(const float* p) { return *reinterpret_cast<const float2*>(p); }

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
  char* kb;      // the layer's K and V base addresses
  char* vb;
};

// WIDE: the row has a K tail (rotary_dim < head_dim) or more V units than
// two per lane; the host picks it, so the common full-rotary shapes carry no
// tail loops.
template <typename T, typename CS, bool NEOX, bool WIDE>
struct RowMover {
  using Table = CS;
  static constexpr int VEC = Elem<T>::kVec;
  static constexpr int NP = NEOX ? VEC : VEC / 2;  // rotation pairs per lane
  const RepositionArgs& a;
  // byte offsets of the token's source and destination slot rows
  int64_t k_src, k_dst, v_src, v_dst;
  // byte offsets inside a slot row (the host keeps a row's span below 2^31):
  // this lane's K unit and its NeoX partner, and its first two V units
  int32_t ko1, ko2, vo0, vo1;
  bool has_v0, has_v1;
  int j, lpr;
  bool same;
  // this lane's first frequency in the token's LDS block of five arrays
  // (cos old, sin old, cos new, sin new, cos^2 + sin^2 of old), each `cstride`
  // floats apart
  const float* coef;
  int cstride;

  __device__ __forceinline__ const T* at(const char* base, int64_t row, int32_t off) const {
    return reinterpret_cast<const T*>(base + row + off);
  }
  __device__ __forceinline__ T* at(char* base, int64_t row, int32_t off) const {
    return reinterpret_cast<T*>(base + row + off);
  }

  template <bool ALIGNED>
  __device__ __forceinline__ RowData load(int layer) const {
    return load_at<ALIGNED>(a.k_ptrs[layer], a.v_ptrs[layer]);
  }

  // the rows of the layer whose K and V buffers start at kbase / vbase
  template <bool ALIGNED>
  __device__ __forceinline__ RowData load_at(uint64_t kbase, uint64_t vbase) const {
    RowData r;
    r.kb = reinterpret_cast<char*>(static_cast<uintptr_t>(kbase));
    r.vb = reinterpret_cast<char*>(static_cast<uintptr_t>(vbase));
    r.k1 = load16<ALIGNED>(at(r.kb, k_src, ko1));
    r.k2 = NEOX ? load16<ALIGNED>(at(r.kb, k_src, ko2)) : make_u32x4(0, 0, 0, 0);
    // without a K tail a NeoX lane moves exactly two V units and a GPT-J lane
    // one (the V row has 2 or 1 units per lane): no per-lane predicate
    if (WIDE ? has_v0 : true) r.v[0] = load16<ALIGNED>(at(r.vb, v_src, vo0));
    if (WIDE ? has_v1 : NEOX) r.v[1] = load16<ALIGNED>(at(r.vb, v_src, vo1));
    return r;
  }

  template <bool ALIGNED>
  __device__ __forceinline__ void finish(const RowData& r) const {
    // V first: it needs no arithmetic, and its registers free up before the
    // rotation's
    if (WIDE ? has_v0 : true) store16<ALIGNED>(at(r.vb, v_dst, vo0), r.v[0]);
    if (WIDE ? has_v1 : NEOX) store16<ALIGNED>(at(r.vb, v_dst, vo1), r.v[1]);
    u32x4 o1 = r.k1, o2 = r.k2;
    if (!same) {
      // two pairs at a time: their ten coefficients are read from LDS just
      // before use, so few registers stay live
      const uint32_t w1[4] = {o1.x, o1.y, o1.z, o1.w};
      const uint32_t w2[4] = {o2.x, o2.y, o2.z, o2.w};
      uint32_t r1[4], r2[4];
#pragma unroll
      for (int k = 0; k < NP; k += 2) {
        // a scheduling fence per chunk keeps the compiler from issuing every
        // chunk's LDS reads up front (which holds all coefficients in
        // registers)
        __builtin_amdgcn_sched_barrier(0);
        const float2 co = lds2(coef + k);
        const float2 so = lds2(coef + cstride + k);
        const float2 cn = lds2(coef + 2 * cstride + k);
        const float2 sn = lds2(coef + 3 * cstride + k);
        const float2 s2 = lds2(coef + 4 * cstride + k);
        float x1[2], x2[2], y1[2], y2[2];
        if (NEOX) {
          // pairs k, k+1: element k (and k+1) of each half
          unpack_two<T>(w1, k, x1);
          unpack_two<T>(w2, k, x2);
        } else {
          // pair k is elements 2k, 2k+1 of the interleaved unit
          float e[4];
          unpack_two<T>(w1, 2 * k, e);
          unpack_two<T>(w1, 2 * k + 2, e + 2);
          x1[0] = e[0];
          x2[0] = e[1];
          x1[1] = e[2];
          x2[1] = e[3];
        }
        rotate(x1[0], x2[0], co.x, so.x, s2.x, cn.x, sn.x, y1[0], y2[0]);
        rotate(x1[1], x2[1], co.y, so.y, s2.y, cn.y, sn.y, y1[1], y2[1]);
        if (NEOX) {
          pack_two<T>(y1, k, r1);
          pack_two<T>(y2, k, r2);
        } else {
          const float e1[2] = {y1[0], y2[0]}, e2[2] = {y1[1], y2[1]};
          pack_two<T>(e1, 2 * k, r1);
          pack_two<T>(e2, 2 * k + 2, r1);
        }
      }
      o1 = make_u32x4(r1[0], r1[1], r1[2], r1[3]);
      if (NEOX) o2 = make_u32x4(r2[0], r2[1], r2[2], r2[3]);
    }
    store16<ALIGNED>(at(r.kb, k_dst, ko1), o1);
    if (NEOX) store16<ALIGNED>(at(r.kb, k_dst, ko2), o2);
    if (!WIDE) return;
    // V units beyond two per lane (wide heads with few rotary units)
    const int v_units_head = a.head_dim / VEC;
    const int v_units_row = a.n_heads * v_units_head;
    for (int c = j + 2 * lpr; c < v_units_row; c += lpr) {
      const int vh = c / v_units_head;
      const int32_t off = static_cast<int32_t>((vh * a.v_stride_head + (c - vh * v_units_head) * VEC) * sizeof(T));
      store16<ALIGNED>(at(r.vb, v_dst, off), load16<ALIGNED>(at(r.vb, v_src, off)));
    }
    // K tail dims [R, D)
    const int t_units_head = (a.head_dim - a.rotary_dim) / VEC;
    const int t_units_row = a.n_heads * t_units_head;
    for (int c = j; c < t_units_row; c += lpr) {
      const int th = c / t_units_head;
      const int32_t off =
          static_cast<int32_t>((th * a.k_stride_head + a.rotary_dim + (c - th * t_units_head) * VEC) * sizeof(T));
      store16<ALIGNED>(at(r.kb, k_dst, off), load16<ALIGNED>(at(r.kb, k_src, off)));
    }
  }
};

// The rows of one token over layers [lbeg, lend): the first layer's K/V
// rows and the token's table rows are loaded together (one round trip), the
// coefficients go to LDS, the one barrier publishes them (waiting for the
// LDS stores only, not for the rows in flight), then each layer is rotated
// and stored, one row in flight per lane (measured faster than prefetching
// the next layer's row: fewer registers, more resident waves).  The loads
// are unconditional -- a lane with no live token reads slot 0's row and
// table row 0, which every pool and table has -- so no load waits behind a
// divergent branch; only the stores are predicated.  Every thread of the
// workgroup reaches the barrier.
template <bool ALIGNED, typename Mover>
__device__ __forceinline__ void move_rows(const RepositionArgs& a, Mover& mv, float* coef, int cstride, int half,
                                          int j, int lpr, bool rotating, bool moving, int64_t old_pos,
                                          int64_t new_pos, int lbeg, int lend, uint64_t kbase, uint64_t vbase) {
  using CS = typename Mover::Table;
  const RowData row = mv.template load_at<ALIGNED>(kbase, vbase);
  const CS* table = static_cast<const CS*>(a.cos_sin);
  const CS* ro = table + (rotating ? old_pos : 0) * a.rope_stride;
  const CS* rn = table + (rotating ? new_pos : 0) * a.rope_stride;
  for (int f = j; f < half; f += lpr) {
    const float co = to_float(ro[f]);
    const float so = to_float(ro[half + f]);
    const float cn = to_float(rn[f]);
    const float sn = to_float(rn[half + f]);
    if (rotating) {
      coef[f] = co;
      coef[cstride + f] = so;
      coef[2 * cstride + f] = cn;
      coef[3 * cstride + f] = sn;
      coef[4 * cstride + f] = co * co + so * so;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (!moving) return;
  mv.template finish<ALIGNED>(row);
  for (int layer = lbeg + 1; layer < lend; ++layer) mv.template finish<ALIGNED>(mv.template load<ALIGNED>(layer));
}

// Workgroup = tokens_per_block consecutive tokens x lanes_per_row lanes, over
// layers_per_block layers of one layer group (token inner: a wave covers
// consecutive tokens of one layer, so slot-adjacent tokens make one
// contiguous span).  Token blocks are numbered fastest, so at any moment the
// device works through a few layers' buffers.  Dynamic LDS holds, per
// token, the five coefficient arrays of its `half` frequencies.  One round
// trip brings the token's list entries, the gate and the layer bases, the
// next both its table rows and its first layer's K/V rows; only the LDS
// coefficients wait at the barrier.
template <typename T, typename CS, bool NEOX, bool WIDE>
__global__ void __launch_bounds__(1024) reposition_vec_kernel(const RepositionArgs a) {
  using Mover = RowMover<T, CS, NEOX, WIDE>;
  constexpr int VEC = Mover::VEC;
  extern __shared__ float4 coef_lds[];
  const int lpr = a.lanes_per_row;
  const int slot = threadIdx.x / lpr;
  const int j = threadIdx.x - slot * lpr;
  // workgroup -> (chunk, layer group, token block), token blocks fastest
  const uint32_t per_chunk = static_cast<uint32_t>(a.chunk_blocks) * static_cast<uint32_t>(a.layer_groups);
  const uint32_t full = static_cast<uint32_t>(a.token_blocks / a.chunk_blocks);
  uint32_t r, rb, first;
  if (blockIdx.x < full * per_chunk) {
    const uint32_t chunk = blockIdx.x / per_chunk;
    r = blockIdx.x - chunk * per_chunk;
    rb = static_cast<uint32_t>(a.chunk_blocks);
    first = chunk * rb;
  } else {  // the last, shorter chunk
    r = blockIdx.x - full * per_chunk;
    first = full * static_cast<uint32_t>(a.chunk_blocks);
    rb = static_cast<uint32_t>(a.token_blocks) - first;
  }
  const uint32_t group = r / rb;
  const int64_t token = static_cast<int64_t>(first + (r - group * rb)) * a.tokens_per_block + slot;
  // group < ceil(n_layers / layers_per_block): the layer range is never empty
  const int lbeg = static_cast<int>(group) * a.layers_per_block;
  const int lend = lbeg + a.layers_per_block < a.n_layers ? lbeg + a.layers_per_block : a.n_layers;
  const int half = a.rotary_dim >> 1;
  const int cstride = coef_stride(half);
  float* coef = reinterpret_cast<float*>(coef_lds) + slot * 5 * cstride;

  // one round of independent loads: the gate, the layer bases and the
  // token's list entries (lanes past the end read the last token's entries)
  // (without a gate the load reads the first source slot, any word will do)
  const int32_t word = __hip_atomic_load(a.gate ? a.gate : a.src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t kbase = a.k_ptrs[lbeg], vbase = a.v_ptrs[lbeg];
  const int64_t tc = token < a.n_tokens ? token : a.n_tokens - 1;
  const int64_t src = a.src[tc];
  const int64_t dst = a.dst[tc];
  const int32_t* pair = a.pairs + tc * a.pair_stride;
  const int64_t old_pos = pair[0];
  const int64_t new_pos = pair[1];
  // every load above is issued before anything waits for one of them (the
  // scheduler would otherwise test the gate first): one round trip.  A
  // closed gate then stops the whole workgroup (the word is the same for
  // every thread) before any K/V row or table row is read.
  __builtin_amdgcn_sched_barrier(0);
  if (a.gate && (word & AKV_STATUS_UNUSABLE) != 0) return;
  const bool live = token < a.n_tokens && !(a.skip_unmapped && (src <= 0 || dst <= 0));
  Mover mv{a};
  mv.same = old_pos == new_pos;
  const bool rotating = live && !mv.same;

  constexpr int64_t B = sizeof(T);
  mv.k_src = (live ? src : 0) * a.k_stride_slot * B;
  mv.k_dst = dst * a.k_stride_slot * B;
  mv.v_src = (live ? src : 0) * a.v_stride_slot * B;
  mv.v_dst = dst * a.v_stride_slot * B;
  mv.lpr = lpr;
  mv.j = j;
  const int h = j / a.units_per_head;
  const int g = j - h * a.units_per_head;
  mv.ko1 = static_cast<int32_t>((h * a.k_stride_head + g * VEC) * B);
  mv.ko2 = static_cast<int32_t>((h * a.k_stride_head + half + g * VEC) * B);
  const int v_units_head = a.head_dim / VEC;
  const int v_units_row = a.n_heads * v_units_head;
  const int c0 = j, c1 = j + lpr;
  mv.has_v0 = c0 < v_units_row;
  mv.has_v1 = c1 < v_units_row;
  const int vh0 = c0 / v_units_head, vh1 = c1 / v_units_head;
  mv.vo0 = static_cast<int32_t>((vh0 * a.v_stride_head + (c0 - vh0 * v_units_head) * VEC) * B);
  mv.vo1 = static_cast<int32_t>((vh1 * a.v_stride_head + (c1 - vh1 * v_units_head) * VEC) * B);
  mv.coef = coef + (NEOX ? g * VEC : g * (VEC / 2));
  mv.cstride = cstride;

  // the workgroup's layers share one form: 16-byte vectors when every base
  // is 16-byte aligned, else element-wise (a uniform branch around the rest)
  bool aligned = ((kbase | vbase) & 15) == 0;
  for (int layer = lbeg + 1; layer < lend; ++layer) aligned &= ((a.k_ptrs[layer] | a.v_ptrs[layer]) & 15) == 0;
  if (aligned)
    move_rows<true>(a, mv, coef, cstride, half, j, lpr, rotating, live, old_pos, new_pos, lbeg, lend, kbase, vbase);
  else
    move_rows<false>(a, mv, coef, cstride, half, j, lpr, rotating, live, old_pos, new_pos, lbeg, lend, kbase,
                     vbase);
}

// Any layout: one thread per (token, layer, head, dim) element.
template <typename T, typename CS>
__global__ void __launch_bounds__(256) reposition_generic_kernel(const RepositionArgs a, int64_t total) {
  const int D = a.head_dim;
  const int H = a.n_heads;
  const int R = a.rotary_dim;
  const int half = R >> 1;
  if (gated(a.gate)) return;
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

// Launch geometry of the vector kernel, measured on MI355X for the 36-layer
// x 8-head x 64 bf16 shape (32 lanes per row) over random and ascending
// slots: 8 tokens x 1 layer per 256-thread workgroup (token blocks fastest)
// beat the earlier 1 token x 36 layers (12 side by side, 3 passes) by 1-1.5%
// on random slots and 7% on ascending ones, and beat 2-32 tokens x 1-4
// layers, several layers side by side, layer groups fastest, and lanes
// reading their coefficients straight from the table instead of LDS.  The
// rule: about 256 threads of consecutive tokens, one layer each.
// The sweep order, measured on MI355X: every layer's workgroup re-reads its
// tokens' cos/sin rows (25% over the K/V reads of a GPT-OSS row), which
// stays cheap while the rows of all tokens stay cached.  So one sweep when
// they fit kSweepTableBytes (the 32k GPT-OSS request's 12064 copies: 6 MB;
// chunks of 4096-12288 tokens measured 0.5-1.5% slower), else chunks of
// kChunkTokens tokens, each swept over every layer before the next (Llama-3
// page-16 copy-on-write, 777k copies and 777 MB of table rows: 61% of HBM
// peak in one sweep, 72 / 75 / 76.7% in chunks of 16384 / 4096 / 1024).
constexpr int64_t kSweepTableBytes = 16ll << 20;
constexpr int64_t kChunkTokens = 1024;
void geometry(RepositionArgs& a) {
  int tokens = 256 / a.lanes_per_row;
  if (tokens < 1) tokens = 1;
  a.tokens_per_block = tokens;
  a.layers_per_block = 1;
}

template <typename T, typename CS>
int launch_typed(RepositionArgs a, int64_t n_tokens, hipStream_t stream, bool vec_ok) {
  constexpr int VEC = Elem<T>::kVec;
  a.n_tokens = n_tokens;
  if (vec_ok) {
    a.units_per_head = a.is_neox ? a.rotary_dim / (2 * VEC) : a.rotary_dim / VEC;
    a.lanes_per_row = a.n_heads * a.units_per_head;
    geometry(a);
    const int threads = a.lanes_per_row * a.tokens_per_block;
    const size_t lds = static_cast<size_t>(a.tokens_per_block) * 5 * coef_stride(a.rotary_dim >> 1) * sizeof(float);
    const bool wide = a.rotary_dim < a.head_dim || a.n_heads * (a.head_dim / VEC) > 2 * a.lanes_per_row;
    void (*kernel)(RepositionArgs) =
        a.is_neox ? (wide ? reposition_vec_kernel<T, CS, true, true> : reposition_vec_kernel<T, CS, true, false>)
                  : (wide ? reposition_vec_kernel<T, CS, false, true> : reposition_vec_kernel<T, CS, false, false>);
    // token blocks in multiples of 8: the dispatcher deals workgroups to the
    // 8 XCDs round robin, so a token block meets the same XCD (and L2) in
    // every layer (the padding blocks hold no live token)
    const int64_t blocks = ((n_tokens + a.tokens_per_block - 1) / a.tokens_per_block + 7) / 8 * 8;
    const int64_t groups = (a.n_layers + a.layers_per_block - 1) / a.layers_per_block;
    const int64_t table_bytes = n_tokens * 2 * a.rotary_dim * static_cast<int64_t>(sizeof(CS));
    const int64_t chunk_tokens = table_bytes <= kSweepTableBytes ? n_tokens : kChunkTokens;
    int64_t chunk = ((chunk_tokens + a.tokens_per_block - 1) / a.tokens_per_block + 7) / 8 * 8;
    if (chunk > blocks) chunk = blocks;
    if (blocks * groups > 0x7fffffffLL)
      return fail(AKV_EINVAL, "akv_reposition_kv_layers: %lld tokens x %d layers exceed one launch",
                  static_cast<long long>(n_tokens), a.n_layers);
    a.token_blocks = static_cast<int32_t>(blocks);
    a.chunk_blocks = static_cast<int32_t>(chunk);
    a.layer_groups = static_cast<int32_t>(groups);
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks * groups)), dim3(threads), lds, stream, a);
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

extern "C" int akv_reposition_kv_layers_gated(const uint64_t* k_ptrs, const uint64_t* v_ptrs,
                                              int32_t n_layers, int32_t kv_dtype, int32_t n_heads,
                                              int32_t head_dim, int32_t rotary_dim, int64_t k_stride_slot,
                                              int64_t k_stride_head, int64_t v_stride_slot,
                                              int64_t v_stride_head, const int32_t* src,
                                              const int32_t* dst, const int32_t* pairs,
                                              int64_t pair_stride, int64_t n_tokens, const void* cos_sin,
                                              int32_t cos_sin_dtype, int64_t rope_stride, int32_t is_neox,
                                              int32_t skip_unmapped, const int32_t* status, void* stream) {
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
  a.gate = status;
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
  // rotary boundary.
  const int vec = 16 / dtype_bytes(kv_dtype);
  bool vec_ok = head_dim % vec == 0 && k_stride_slot % vec == 0 && k_stride_head % vec == 0 &&
                v_stride_slot % vec == 0 && v_stride_head % vec == 0 &&
                (is_neox ? rotary_dim % (2 * vec) == 0 : rotary_dim % vec == 0);
  if (vec_ok) {
    const int units = is_neox ? rotary_dim / (2 * vec) : rotary_dim / vec;
    if (static_cast<int64_t>(n_heads) * units > 1024) vec_ok = false;
    // byte offsets inside one slot row are 32-bit in the vector kernel
    const int64_t row_span = (static_cast<int64_t>(n_heads) * (k_stride_head > v_stride_head ? k_stride_head
                                                                                              : v_stride_head) +
                              head_dim) * dtype_bytes(kv_dtype);
    if (k_stride_head < 0 || v_stride_head < 0 || row_span >= (1LL << 31)) vec_ok = false;
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

extern "C" int akv_reposition_kv_layers(const uint64_t* k_ptrs, const uint64_t* v_ptrs,
                                        int32_t n_layers, int32_t kv_dtype, int32_t n_heads,
                                        int32_t head_dim, int32_t rotary_dim, int64_t k_stride_slot,
                                        int64_t k_stride_head, int64_t v_stride_slot,
                                        int64_t v_stride_head, const int32_t* src,
                                        const int32_t* dst, const int32_t* pairs,
                                        int64_t pair_stride, int64_t n_tokens, const void* cos_sin,
                                        int32_t cos_sin_dtype, int64_t rope_stride, int32_t is_neox,
                                        int32_t skip_unmapped, void* stream) {
  return akv_reposition_kv_layers_gated(k_ptrs, v_ptrs, n_layers, kv_dtype, n_heads, head_dim, rotary_dim,
                                        k_stride_slot, k_stride_head, v_stride_slot, v_stride_head, src, dst,
                                        pairs, pair_stride, n_tokens, cos_sin, cos_sin_dtype, rope_stride, is_neox,
                                        skip_unmapped, nullptr, stream);
}
