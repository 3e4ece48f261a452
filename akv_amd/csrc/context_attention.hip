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
// Workgroup = (block of R / G query tokens, KV head g, segment), KV head
// fastest in the grid (workgroup id mod 8 picks the XCD: with 8 KV heads each
// XCD's L2 serves one head's K/V), with the
// G q heads of the group packed as rows: row r = token * G + head; R = 512
// rows at head_dim 64 (8 waves x 64 rows, so each wave's reads of a K/V tile
// from LDS feed 64 rows), 256 at head_dim 128 (8 waves x 32 rows); one
// workgroup per CU, two waves per SIMD, so every K/V tile a CU stages from
// L2 feeds all of its rows.  Per
// tile of 128 keys (full layers at head_dim 64) or 64 (K and V key-major in
// LDS with XOR-swizzled 16 B chunks, double buffered; the next tile's rows
// stream straight from HBM into LDS with global_load_lds_dwordx4 -- no
// staging registers -- and the slots of the tile after it are fetched, all
// during this tile's math), in 32-key quarters, for a wave's W rows:
//   S^T[32 keys x W rows] = K . Q^T           v_mfma_f32_16x16x32_bf16
//   P^T = 2^(scale log2(e) S^T - m) in bf16   (one fp32 fma per score: Q
//     stays exact -- folding the scale into a bf16 Q costs several times
//     the tolerance once the scores spread over ~40 in the log2 domain)
//   l[rows] += 1^T . P^T                      (row sums of the same bf16 P)
//   O^T[D x W rows] += V^T . P^T              v_mfma_f32_16x16x32_bf16
// Online softmax without per-tile maxima: a row's running maximum m comes
// from exact row maxima (moving only when a quarter exceeds it by 2^8)
// while some row of the wave has seen no key, then stays put.  After each
// tile the weight sums are checked: one past 2^32 is renormalised by a power
// of two; one past 2^64 (a score ~58 above m, or inf) may have overflowed O,
// and the workgroup restarts its keys with exact maxima on every tile.
// P^T leaves the first MFMA in the B-operand layout of the second (any
// consistent split of the 32-long k axis over lanes gives the same product:
// lane l uses keys 4(l/16)+i of two 16-key subtiles); V^T comes from the
// key-major tile through ds_read_b64_tr_b16.  Tiles wholly inside every
// row's causal and window range skip the mask.
//
// Two instances of each shape: the plain one (head_dim 64 or 128, the group
// a power of two, no logit cap) and the general one, which pads a token's
// rows to a power-of-two group (padding rows keep Q = 0 and store nothing),
// runs heads narrower than the tile with the unloaded dims zero in LDS, and
// caps scaled scores at cap tanh(s / cap) before the mask.
//
// Lane layouts (verified on gfx950): v_mfma_f32_16x16x32_bf16 -- lane l
// supplies A[l%16][k(l,i)], B[k(l,i)][l%16] for i < 8 and holds
// D[4(l/16)+i][l%16]; ds_read_b64_tr_b16 -- within each 16-lane group, lane
// j receives element j%4 of the 8-byte rows read by lanes j/4 + 4i, i < 4.
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
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// 16-row subtiles per wave: 4 at head_dim 64 (each wave's K/V tile reads
// from LDS feed 64 rows), 2 at head_dim 128 (register budget)
constexpr int sub_tiles(int d) { return d == 64 ? 4 : 2; }
// 8 waves: the register budget allows two waves per SIMD, so a workgroup of
// 8 fills the CU alone and its K/V tiles feed twice the rows of two 4-wave
// workgroups (half the tile loads per flop, and twice the math per tile to
// hide each tile's load behind)
constexpr int kWaves = 8;
constexpr int rows_per_block(int d) { return kWaves * 16 * sub_tiles(d); }  // (token, head) rows
constexpr int kThreads = 64 * kWaves;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.f;  // log2-domain slack before an exact maximum moves
constexpr float kBig = 4294967296.f;  // 2^32: a weight sum above it is renormalised
constexpr float kHuge = 18446744073709551616.f;  // 2^64: above it the product may have overflowed

struct CtxArgs {
  const __bf16* q;
  const __bf16* k_ext;
  const __bf16* v_ext;
  const __bf16* k_pool;
  const __bf16* v_pool;
  const void* qo_indptr;
  const void* kv_indptr;
  const void* kv_indices;
  const void* q_pos;
  const void* kv_pos;
  const float* sinks;
  void* out;
  // element strides (checked to fit 32 bits on the host)
  int32_t q_st, q_sh, ke_st, ke_sh, ve_st, ve_sh, kp_ss, kp_sh, vp_ss, vp_sh, o_st, o_sh;
  int32_t indptr_i64;
  int32_t window;
  float scale_log2;
  int32_t out_f32;
  int32_t group, group_shift, tokens_per_block, kv_heads;
  int32_t head_dim;   // head dims in use (<= the kernel's D; the rest are zero)
  float cap, cap_log2;  // logit cap (scores -> cap tanh(score / cap)), cap log2(e)
};

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Maximum over the four lanes col, col+16, col+32, col+48 of each 16-lane
// column group, on the VALU: v_permlane16_swap / v_permlane32_swap exchange
// rows of 16 (32) lanes, so max(swapped pair) = max(own, partner).
// v_max3_f32 / v_max_f32 without the canonicalising moves the compiler adds
// around fmaxf of matrix-core results.  Only the softmax's range uses these
// maxima: a NaN score still reaches the output through exp2 and the MFMAs.
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ float max2(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

__device__ __forceinline__ float row_max(float x) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  const auto r16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  // copy the pair out before the bit casts: a bit cast of a vector element
  // reference reads element 0
  const uint32_t a0 = r16[0], a1 = r16[1];
  x = max2(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
  const uint32_t c = __builtin_bit_cast(uint32_t, x);
  const auto r32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  const uint32_t c0 = r32[0], c1 = r32[1];
  return max2(__builtin_bit_cast(float, c0), __builtin_bit_cast(float, c1));
}

__device__ __forceinline__ u32x4 load16(const __bf16* p) {
  return *((const global_u32x4*)p);
}

// One of the two LDS tile buffers.  They are separate objects, named
// statically in each half of the unrolled tile loop, so the compiler sees
// that this tile's LDS reads never touch the other buffer that the next
// tile's direct loads are filling (no wait on those loads mid-tile in the
// 64-key instances; the rolled quarter loop of the 128-key ones still gets
// a wait before its transposing reads, which measured free).
template <int D, int KEYS>
struct TileLds {
  __bf16 k[KEYS][D];   // key-major K tile, 16 B chunks swizzled per row (swz_k)
  __bf16 v[KEYS][D];   // key-major V tile, read transposed (ds_read_b64_tr_b16), swizzled (swz_v)
  int32_t pos[KEYS];   // key positions relative to the block's first query
};

// Chunk swizzles: logical 16 B chunk c of row r lives at chunk c ^ swz(r).
// K (16 B operand reads, 16 rows per lane group): distinct banks for the 16
// rows of a read.  V (8 B transposed reads, 4 rows x 32 B per 16 lanes, 8
// rows per 32 lanes): bit 0 clear so a row's chunk pair stays adjacent, and
// distinct bank groups for 8 consecutive rows.  At head_dim 64 a row is half
// the 64 banks (rows of opposite parity use opposite halves).
template <int D>
__device__ __forceinline__ int swz_k(int r) { return D == 64 ? (r >> 1) & 7 : r & 15; }
template <int D>
__device__ __forceinline__ int swz_v(int r) { return D == 64 ? r & 6 : (r & 7) << 1; }

typedef __attribute__((address_space(3))) void lds_void;

constexpr int32_t kFar = 1 << 30;  // relative positions are clamped to [-kFar, kFar]

__device__ __forceinline__ int32_t rel_pos(int64_t p, int64_t base) {
  const int64_t r = p - base;
  return static_cast<int32_t>(r < -kFar ? -kFar : (r > kFar ? kFar : r));
}

// KEYS keys per tile: 128 for full layers at head_dim 64 (half the tile
// barriers, staging and commits per key), 64 for windowed layers (less of a
// tile outside the window) and at head_dim 128 (measured faster than 128 there)
// GEN: the general instance -- logit caps, heads narrower than D (the dims
// past head_dim zero in the tiles), groups padded to a power of two; the
// plain instance takes none of these checks.
template <int D, int KEYS, typename IdxT, typename PosT, bool POS, bool GEN>
__global__ void __launch_bounds__(kThreads, 2) context_attention_kernel(const CtxArgs a) {
  constexpr int kSub = sub_tiles(D);
  constexpr int kKeys = KEYS;
  constexpr int kChunks = D / 8;               // 16 B chunks per key row
  constexpr int kKSteps = D / 32;              // MFMA k-steps over head dims
  constexpr int kDTiles = D / 16;              // O^T row tiles
  __shared__ __attribute__((aligned(16))) TileLds<D, KEYS> tile0, tile1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS block bases in SGPRs
  const int col = lane & 15;
  const int quad = lane >> 4;
  const int seg = blockIdx.z;
  const bool i64 = a.indptr_i64;
  const int64_t qo0 = load_index(a.qo_indptr, i64, seg);
  const int32_t qlen = static_cast<int32_t>(load_index(a.qo_indptr, i64, seg + 1) - qo0);
  const int G = a.group;                         // q heads per KV head
  const int gmask = (1 << a.group_shift) - 1;    // rows per token: G padded to a power of two
  const int T = a.tokens_per_block;
  const int hd = GEN ? a.head_dim : D;
  const bool cap = GEN && a.cap > 0.f;
  // the score's log2-domain multiplier: with a cap the scores are capped
  // (and scaled) before the softmax, which then takes them as they are
  const float mult = cap ? 1.f : a.scale_log2;
  // KV head fastest: workgroup id mod 8 picks the XCD, so with 8 KV heads
  // every XCD streams one head's K/V through its own L2.  Token blocks run
  // last-first: the last blocks see the most causal keys, and starting them
  // first shortens the tail of the launch.
  const int g = static_cast<int>(blockIdx.x % static_cast<unsigned>(a.kv_heads));
  const int32_t t0 = static_cast<int32_t>(gridDim.x / static_cast<unsigned>(a.kv_heads) - 1 -
                                          blockIdx.x / static_cast<unsigned>(a.kv_heads)) * T;
  if (t0 >= qlen) return;
  const int64_t kv0 = load_index(a.kv_indptr, i64, seg);
  // without prefix indices there is no prefix, whatever kv_indptr says
  const int32_t plen =
      a.kv_indices ? static_cast<int32_t>(load_index(a.kv_indptr, i64, seg + 1) - kv0) : 0;
  // segment-local views
  const PosT* qpos = static_cast<const PosT*>(a.q_pos) + qo0;
  const PosT* kpos = static_cast<const PosT*>(a.kv_pos) + kv0;
  const IdxT* slots = static_cast<const IdxT*>(a.kv_indices) + kv0;
  const __bf16* kext = a.k_ext + qo0 * a.ke_st + g * a.ke_sh;
  const __bf16* vext = a.v_ext + qo0 * a.ve_st + g * a.ve_sh;
  const __bf16* kpool = a.k_pool + g * a.kp_sh;
  const __bf16* vpool = a.v_pool + g * a.vp_sh;
  const char* kext_b = reinterpret_cast<const char*>(kext);
  const char* vext_b = reinterpret_cast<const char*>(vext);
  const char* kpool_b = reinterpret_cast<const char*>(kpool);
  const char* vpool_b = reinterpret_cast<const char*>(vpool);
  const uint64_t ke_sb = 2u * static_cast<uint32_t>(a.ke_st), ve_sb = 2u * static_cast<uint32_t>(a.ve_st);
  const uint64_t kp_sb = 2u * static_cast<uint32_t>(a.kp_ss), vp_sb = 2u * static_cast<uint32_t>(a.vp_ss);
  auto qpos_of = [&](int32_t i) -> int64_t {  // position of query i of the segment
    if constexpr (POS) return static_cast<int64_t>(qpos[i]);
    return static_cast<int64_t>(plen) + i;
  };
  auto kpos_of = [&](int32_t j) -> int64_t {  // position of prefix key j
    if constexpr (POS) return static_cast<int64_t>(kpos[j]);
    return static_cast<int64_t>(j);
  };
  const int64_t qbase = qpos_of(t0);
  const int32_t e_hi = qlen < t0 + T ? qlen : t0 + T;  // extend keys [e_lo, e_hi)
  const int32_t last_rel = rel_pos(qpos_of(e_hi - 1), qbase);

  // keys below qbase - window are outside every row's window
  int32_t p_lo = 0, e_lo = 0;
  if (a.window >= 0) {
    const int64_t first = qbase - a.window;
    int32_t lo = 0, hi = plen;
    while (lo < hi) {
      const int32_t mid = (lo + hi) >> 1;
      if (kpos_of(mid) < first) lo = mid + 1; else hi = mid;
    }
    p_lo = lo;
    lo = 0;
    hi = t0;
    while (lo < hi) {
      const int32_t mid = (lo + hi) >> 1;
      if (qpos_of(mid) < first) lo = mid + 1; else hi = mid;
    }
    e_lo = lo;
  }
  const int n_pref = (plen - p_lo + kKeys - 1) / kKeys;
  const int n_tiles = n_pref + (e_hi - e_lo + kKeys - 1) / kKeys;
  auto tile_base = [&](int it) -> int32_t {
    return it < n_pref ? p_lo + it * kKeys : e_lo + (it - n_pref) * kKeys;
  };

  // this lane's rows: row subtile s covers rows wave * 16 kSub + 16s + col,
  // row r = (token r >> group_shift, q head g G + r % G); the rows'
  // positions relative to qbase wait in LDS for the masked tiles
  __shared__ int32_t rel_rows[rows_per_block(D)];
  auto row_of = [&](int s) { return wave * (16 * kSub) + 16 * s + col; };
  bf16x8 qop[kSub][kKSteps];
#pragma unroll
  for (int s = 0; s < kSub; ++s) {
    const int r = row_of(s);
    const int tl = r >> a.group_shift;
    const int hl = r & gmask;
    const int head = g * G + hl;
    const bool tok = t0 + tl < qlen;
    // a padding row (hl >= G) keeps Q = 0 and is never stored
    const bool ok = tok && (!GEN || hl < G);
    if (quad == 0) rel_rows[r] = tok ? rel_pos(qpos_of(t0 + tl), qbase) : last_rel;
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      u32x4 w = {0u, 0u, 0u, 0u};
      // head dims past hd are zero
      if (ok && (!GEN || 8 * (4 * ks + quad) < hd))
        w = load16(a.q + (qo0 + t0 + tl) * a.q_st + static_cast<int64_t>(head) * a.q_sh + 32 * ks + 8 * quad);
      qop[s][ks] = __builtin_bit_cast(bf16x8, w);
    }
  }

  // tile staging straight into LDS (global_load_lds_dwordx4: lane l of a
  // wave instruction fills bytes 16 l of a 1 KiB block).  Block b of a tile
  // holds rows kRowsPerBlock b ..; lane l writes row kRowsPerBlock b + l /
  // kChunks at chunk position l % kChunks, i.e. logical chunk (l % kChunks)
  // ^ swz(row) of that key, which it loads.  Each wave fills kBlocksPerWave
  // blocks of K and of V.  Prefix slots are fetched one tile ahead.
  constexpr int kRowsPerBlock = 1024 / (2 * D);
  constexpr int kBlocksPerWave = kKeys / kRowsPerBlock / kWaves;
  static_assert(kBlocksPerWave >= 1 && kBlocksPerWave * kRowsPerBlock * kWaves == kKeys, "tile split over waves");
  static_assert(kThreads >= kKeys, "one thread per key position");
  // slot indices are below 2^32 (a pool of 2^32 slots of one 64-wide bf16
  // head is 512 GiB): int64 indices address rows through their low 32 bits
  uint32_t slot[kBlocksPerWave];
  int64_t preg = 0;  // raw position of key tid of the staged tile
  bool pvalid = false;
  const int my_row = lane / kChunks;   // row within a block
  const int my_pos = lane % kChunks;   // chunk position within the row
  auto fetch_slots = [&](int it) {
    // keys past the prefix read the last prefix row (finite data, masked out)
    const int32_t base = tile_base(it);
#pragma unroll
    for (int u = 0; u < kBlocksPerWave; ++u) {
      const int32_t j = base + (kBlocksPerWave * wave + u) * kRowsPerBlock + my_row;
      slot[u] = static_cast<uint32_t>(slots[j < plen ? j : plen - 1]);
    }
  };
  auto stage = [&](int it, TileLds<D, KEYS>& t) {
    // branch-free: keys past the end read the last valid row (masked out later)
    const bool ext = it >= n_pref;
    const int32_t base = tile_base(it);
#pragma unroll
    for (int u = 0; u < kBlocksPerWave; ++u) {
      const int blk = kBlocksPerWave * wave + u;
      const int r = blk * kRowsPerBlock + my_row;
      const int ck = my_pos ^ swz_k<D>(r), cv = my_pos ^ swz_v<D>(r);
      const char *krow, *vrow;
      if (ext) {
        const int32_t j = base + r;
        const uint64_t off = static_cast<uint32_t>(j < e_hi ? j : e_hi - 1);
        krow = kext_b + off * ke_sb;
        vrow = vext_b + off * ve_sb;
      } else {
        const uint64_t so = slot[u];
        krow = kpool_b + so * kp_sb;
        vrow = vpool_b + so * vp_sb;
      }
      if (!GEN || hd == D) {
        __builtin_amdgcn_global_load_lds(krow + 16 * ck, (lds_void*)(&t.k[blk * kRowsPerBlock][0]), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vrow + 16 * cv, (lds_void*)(&t.v[blk * kRowsPerBlock][0]), 16, 0, 0);
      } else {
        // narrower heads: chunks past hd are not loaded (they stay zero)
        if (8 * ck < hd)
          __builtin_amdgcn_global_load_lds(krow + 16 * ck, (lds_void*)(&t.k[blk * kRowsPerBlock][0]), 16, 0, 0);
        if (8 * cv < hd)
          __builtin_amdgcn_global_load_lds(vrow + 16 * cv, (lds_void*)(&t.v[blk * kRowsPerBlock][0]), 16, 0, 0);
      }
    }
    // key positions matter only to a window (causal masking is by index)
    if (a.window >= 0 && tid < kKeys) {
      // loaded now, converted at commit: no wait on the tile's row loads here
      const int32_t j = base + tid;
      const int32_t end = ext ? e_hi : plen;
      pvalid = j < end;
      const int32_t jc = pvalid ? j : end - 1;
      preg = ext ? qpos_of(jc) : kpos_of(jc);
    }
  };
  // positions of the staged tile, then wait for its direct loads (vmcnt) so
  // the barrier that follows publishes the whole tile
  auto commit = [&](TileLds<D, KEYS>& t) {
    // (without a window every key's position reads 0, which the mask admits)
    if (tid < kKeys) t.pos[tid] = a.window < 0 ? 0 : (pvalid ? rel_pos(preg, qbase) : kFar);
    __builtin_amdgcn_s_waitcnt(0);
  };

  f32x4 oacc[kDTiles][kSub];
  // per row: the negated running maximum -m (log2 domain; 0 while the row
  // has seen no key) and the running sum of the bf16 weights (4 equal
  // copies); a row with a zero sum has seen no key
  float neg_m[kSub];
  f32x4 lacc[kSub];
  auto clear_rows = [&]() {
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
      neg_m[s] = 0.f;
      lacc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) oacc[dt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  clear_rows();
  // some row of this wave has seen no key yet (uniform): tiles take the
  // exact row maxima until every row has a maximum
  bool unset = true;
  // after a restart every tile takes the exact maxima (uniform)
  bool exact_all = false;
  __shared__ int32_t restart_flag;
  if (tid == 0) restart_flag = 0;
  const bf16x8 kOnes = {__bf16(1.f), __bf16(1.f), __bf16(1.f), __bf16(1.f),
                        __bf16(1.f), __bf16(1.f), __bf16(1.f), __bf16(1.f)};

  if (GEN && hd < D) {
    // narrower heads: the tiles' chunks past hd are never loaded; zero them
    // once.  The stores cover every chunk, loaded ones too, so they must
    // land before any wave's direct loads into tile 0: barrier first.
    constexpr int kWords = KEYS * D / 8;  // 16 B chunks per array
    for (int i = tid; i < 4 * kWords; i += kThreads) {
      __bf16* arr = i < kWords ? &tile0.k[0][0] : i < 2 * kWords ? &tile0.v[0][0]
                  : i < 3 * kWords ? &tile1.k[0][0] : &tile1.v[0][0];
      reinterpret_cast<u32x4*>(arr)[i % kWords] = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
  }
  if (n_pref > 0) fetch_slots(0);
  stage(0, tile0);
  if (1 < n_pref) fetch_slots(1);
  commit(tile0);
  __syncthreads();
  // tile it from cur while tile it + 1 streams into nxt
  auto step = [&](int it, TileLds<D, KEYS>& cur, TileLds<D, KEYS>& nxt) {
    if (it + 1 < n_tiles) {
      stage(it + 1, nxt);
      if (it + 2 < n_pref) fetch_slots(it + 2);
    }
    const bool ext = it >= n_pref;
    const int32_t base = tile_base(it);
    const int32_t left = (ext ? e_hi : plen) - base;
    const int count = left < kKeys ? left : kKeys;
    // masking is needed for a partial tile, keys past the block's first
    // query (causal), or keys older than the last query's window
    const bool masked = count < kKeys || (ext && base + kKeys - 1 > t0) ||
                        (a.window >= 0 && __builtin_amdgcn_readfirstlane(cur.pos[0]) < last_rel - a.window);
    const bool exact = unset || exact_all;

    // The tile in quarters of 32 keys (kk), each complete before the next:
    //   S^T = K . Q^T
    //   P^T = 2^(scale log2(e) S^T - m) in bf16  (the B operand of both products)
    //   l += 1^T . P^T         (row sums of the same bf16 weights on the
    //                           matrix cores: O stays a convex combination)
    //   O^T += V^T . P^T
    // Masked tiles add the mask (masked scores become -inf in place: exp2 ->
    // 0); exact tiles the row maxima (column of S^T: lanes col, col+16,
    // col+32, col+48): a row's maximum moves when the half exceeds it by more
    // than kLazy (a row that has seen no key: on any visible key), scaling O
    // and l by 2^-move.  Both stay runtime branches: a branch-free fast tile
    // lets the scheduler hoist the second half's reads and products into
    // the first half and spill.
    auto half = [&](int kk) {
      f32x4 sh[2][kSub];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kt = 2 * kk + j;
        const int krow = 16 * kt + col;
#pragma unroll
        for (int ks = 0; ks < kKSteps; ++ks) {
          const bf16x8 kop = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const u32x4*>(&cur.k[krow][8 * ((4 * ks + quad) ^ swz_k<D>(krow))]));
#pragma unroll
          for (int s = 0; s < kSub; ++s)
            sh[j][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[s][ks],
                                                               ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : sh[j][s], 0, 0, 0);
        }
      }
      if (cap) {
        // capped logits: cap tanh(scale s / cap), in the log2 domain, before
        // the mask (a masked score stays -inf); tanh(x) = 1 - 2 / (1 + e^2x).
        // The cap of SGLang's extend kernel, which the reference hands the
        // layer's cap (akv/system/sglang.patch:2437,2459): scale, then cap.
        // Sinks are not capped.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int s = 0; s < kSub; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float e2x = __builtin_amdgcn_exp2f(sh[j][s][i] * a.scale_log2 * (2.f / a.cap));
              sh[j][s][i] = a.cap_log2 * (1.f - 2.f * __builtin_amdgcn_rcpf(1.f + e2x));
            }
      }
      if (masked) {
#pragma unroll
        for (int s = 0; s < kSub; ++s) {
          // causal: key index <= the row's token; window: key pos >= row pos - W
          const int r = row_of(s);
          const int32_t climit = ext ? t0 + (r >> a.group_shift) - base : kKeys;
          const int32_t last = climit < count - 1 ? climit : count - 1;
          const int32_t thr = a.window >= 0 ? rel_rows[r] - a.window : -kFar - 1;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int k0 = 16 * (2 * kk + j) + 4 * quad;
            const i32x4 kp = *reinterpret_cast<const i32x4*>(&cur.pos[k0]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const bool vis = (k0 + i <= last) & (kp[i] >= thr);
              sh[j][s][i] = vis ? sh[j][s][i] : -INFINITY;
            }
          }
        }
      }
      if (exact) {
#pragma unroll
        for (int s = 0; s < kSub; ++s) {
          // 8 values in 4 three-input maxima, then across the lane groups
          const float m0 = max3(sh[0][s][0], sh[0][s][1], sh[0][s][2]);
          const float m1 = max3(sh[0][s][3], sh[1][s][0], sh[1][s][1]);
          float mx = max3(m0, m1, max3(sh[1][s][2], sh[1][s][3], -INFINITY));
          mx = row_max(mx);  // -inf when the row sees nothing here
          // the half's largest exponent, t - m in the log2 domain
          const float top = fmaf(mx, mult, neg_m[s]);
          const bool seen = lacc[s][0] != 0.f;
          const bool bump = seen ? top > kLazy : mx > -INFINITY;
          if (__builtin_amdgcn_ballot_w64(bump)) {
            const float alpha = bump && seen ? __builtin_amdgcn_exp2f(-top) : 1.f;
            lacc[s] *= alpha;
#pragma unroll
            for (int dt = 0; dt < kDTiles; ++dt) oacc[dt][s] *= alpha;
            neg_m[s] = bump ? -(mx * mult) : neg_m[s];
          }
        }
      }
      bf16x8 pop[kSub];
#pragma unroll
      for (int s = 0; s < kSub; ++s) {
        f32x4 e0, e1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          e0[i] = __builtin_amdgcn_exp2f(fmaf(sh[0][s][i], mult, neg_m[s]));
          e1[i] = __builtin_amdgcn_exp2f(fmaf(sh[1][s][i], mult, neg_m[s]));
        }
        const bf16x4 b0 = __builtin_convertvector(e0, bf16x4);
        const bf16x4 b1 = __builtin_convertvector(e1, bf16x4);
        pop[s] = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int s = 0; s < kSub; ++s) lacc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kOnes, pop[s], lacc[s], 0, 0, 0);
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) {
        // transposing read: lane col of group quad receives V[key][16dt + col]
        // for keys 32kk + 4 quad + i (i < 4), then 32kk + 16 + 4 quad + i;
        // source lane col supplies row key0 + col / 4, dims 16dt + 4 (col % 4) ..+3
        // (logical element 16dt + 4(col%4) = chunk 2dt + (col%4)/2, half col%2)
        const int vr0 = 32 * kk + 4 * quad + (col >> 2), vr1 = vr0 + 16;
        const int vc = 2 * dt + ((col & 3) >> 1), vh = 4 * (col & 1);
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)&cur.v[vr0][8 * (vc ^ swz_v<D>(vr0)) + vh]);
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)&cur.v[vr1][8 * (vc ^ swz_v<D>(vr1)) + vh]);
        const bf16x8 vop = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int s = 0; s < kSub; ++s)
          oacc[dt][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[s], oacc[dt][s], 0, 0, 0);
      }
    };
    if constexpr (kKeys == 64) {
      half(0);
      half(1);
    } else {
      // rolled: unrolled, the four quarters' operand reads crowd the registers
#pragma nounroll
      for (int kk = 0; kk < kKeys / 32; ++kk) half(kk);
    }

    // Without maxima the weights' sums are the check: a sum above kBig (a
    // score ~26 above the maximum, or slow growth over many tiles) is
    // renormalised by a power of two (exact); one above kHuge (a score ~58
    // above the maximum, inf included) may have overflowed O: the workgroup
    // restarts its keys with exact maxima on every tile.  NaN sums pass both
    // tests: NaN inputs reach the output.
    bool big = false, huge = false;
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
      big |= lacc[s][0] > kBig;
      huge |= lacc[s][0] > kHuge;
    }
    if (__builtin_amdgcn_ballot_w64(big)) {
      if (!exact && __builtin_amdgcn_ballot_w64(huge)) restart_flag = 1;
      // sum -> [1/2, 1): O and the sum by 2^-e, the maximum up by e
#pragma unroll
      for (int s = 0; s < kSub; ++s) {
        const int e = lacc[s][0] > kBig ? __builtin_amdgcn_frexp_expf(lacc[s][0]) : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) lacc[s][i] = __builtin_amdgcn_ldexpf(lacc[s][i], -e);
#pragma unroll
        for (int dt = 0; dt < kDTiles; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) oacc[dt][s][i] = __builtin_amdgcn_ldexpf(oacc[dt][s][i], -e);
        neg_m[s] -= static_cast<float>(e);
      }
    }
    if (unset) {
      bool none = false;
#pragma unroll
      for (int s = 0; s < kSub; ++s) none |= lacc[s][0] == 0.f;
      unset = __builtin_amdgcn_ballot_w64(none) != 0;
    }
    if (it + 1 < n_tiles) commit(nxt);
    __syncthreads();
  };
  // a restart (decided before the tile's barrier, read after it by every
  // wave) starts the keys again from tile 0 with exact maxima; no load is in
  // flight after a barrier and neither buffer is still being read
  auto restart_flag_set = [&]() -> bool {
    return !exact_all && __builtin_amdgcn_readfirstlane(*static_cast<volatile int32_t*>(&restart_flag));
  };
  auto restarted = [&]() -> bool {
    if (!restart_flag_set()) return false;
    exact_all = true;
    unset = true;
    clear_rows();
    if (n_pref > 0) fetch_slots(0);
    stage(0, tile0);
    if (1 < n_pref) fetch_slots(1);
    commit(tile0);
    __syncthreads();
    return true;
  };
  for (int it = 0; it < n_tiles; it += 2) {
    step(it, tile0, tile1);
    // a restart after the first half skips the second
    if (it + 1 < n_tiles && !restart_flag_set()) step(it + 1, tile1, tile0);
    if (restarted()) it = -2;
  }

  // normalise with the sink; store
#pragma unroll
  for (int s = 0; s < kSub; ++s) {
    float l = lacc[s][0];
    float scale = 1.f;
    const int hl = row_of(s) & gmask;
    if (a.sinks) {
      const float m_run = l != 0.f ? -neg_m[s] : -INFINITY;
      const float sink = a.sinks[g * G + (GEN && hl >= G ? G - 1 : hl)] * kLog2e;
      const float m_f = fmaxf(m_run, sink);
      scale = m_run == -INFINITY ? 0.f : exp2f(m_run - m_f);
      l = l * scale + exp2f(sink - m_f);
    }
    const float inv = l > 0.f ? scale / l : 0.f;
    const int32_t row_token = row_of(s) >> a.group_shift, row_head = g * G + hl;
    if (t0 + row_token >= qlen || (GEN && hl >= G)) continue;
    const int64_t at =
        (qo0 + t0 + row_token) * a.o_st + static_cast<int64_t>(row_head) * a.o_sh + 4 * quad;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) {
      if (GEN && 16 * dt + 4 * quad >= hd) continue;
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

template <int D, int KEYS, typename IdxT, bool GEN>
void launch_pos(int pos, dim3 grid, hipStream_t st, const CtxArgs& a) {
  // pos: 0 none, 1 int32, 2 int64
  if (pos == 2)
    hipLaunchKernelGGL((context_attention_kernel<D, KEYS, IdxT, int64_t, true, GEN>), grid, dim3(kThreads), 0, st, a);
  else if (pos == 1)
    hipLaunchKernelGGL((context_attention_kernel<D, KEYS, IdxT, int32_t, true, GEN>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((context_attention_kernel<D, KEYS, IdxT, int64_t, false, GEN>), grid, dim3(kThreads), 0, st,
                       a);
}

template <int D, int KEYS, typename IdxT>
void launch_cap(int pos, dim3 grid, hipStream_t st, const CtxArgs& a) {
  // the general instance for caps, narrower heads and padded groups
  if (a.cap > 0.f || a.head_dim != D || a.group != (1 << a.group_shift))
    launch_pos<D, KEYS, IdxT, true>(pos, grid, st, a);
  else
    launch_pos<D, KEYS, IdxT, false>(pos, grid, st, a);
}

template <int D, int KEYS>
void launch_idx(bool idx64, int pos, dim3 grid, hipStream_t st, const CtxArgs& a) {
  if (idx64)
    launch_cap<D, KEYS, int64_t>(pos, grid, st, a);
  else
    launch_cap<D, KEYS, int32_t>(pos, grid, st, a);
}

void launch_typed(int head_dim, bool idx64, int pos, dim3 grid, hipStream_t st, const CtxArgs& a) {
  if (head_dim > 64)
    launch_idx<128, 64>(idx64, pos, grid, st, a);
  else if (a.window >= 0)
    launch_idx<64, 64>(idx64, pos, grid, st, a);
  else
    launch_idx<64, 128>(idx64, pos, grid, st, a);
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
                                     float scale, float logit_cap, void* out, int32_t out_dtype,
                                     int64_t out_stride_t, int64_t out_stride_h, int64_t max_query_len,
                                     void* stream) {
  using namespace akv;
  if (n_segments < 0 || max_query_len < 0) return fail(AKV_EINVAL, "akv_context_attention: negative size");
  if (n_segments == 0 || max_query_len == 0) return AKV_OK;
  // heads of up to 128 dims in 16-byte chunks: the kernel's 64- or 128-dim
  // tiles with the dims past head_dim zero
  if (head_dim < 8 || head_dim > 128 || head_dim % 8 != 0)
    return fail(AKV_EINVAL, "akv_context_attention: head_dim %d (supported: multiples of 8 up to 128)", head_dim);
  // a block's rows are (token, q head) pairs with the group padded to a
  // power of two (at most 128 q heads per KV head); a row packs its q head
  // into 15 bits
  if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0 || q_heads / kv_heads > 128 || q_heads > 32767)
    return fail(AKV_EINVAL, "akv_context_attention: %d q heads over %d KV heads (at most 128 per KV head)",
                q_heads, kv_heads);
  if (!(logit_cap >= 0.f) || !std::isfinite(logit_cap))
    return fail(AKV_EINVAL, "akv_context_attention: logit_cap must be 0 (none) or positive and finite");
  if (!valid_index_dtype(indptr_dtype) || !valid_index_dtype(indices_dtype) ||
      !valid_index_dtype(positions_dtype))
    return fail(AKV_EINVAL, "akv_context_attention: index vectors must be int32 or int64");
  if (out_dtype != AKV_BF16 && out_dtype != AKV_F32)
    return fail(AKV_EINVAL, "akv_context_attention: output must be bf16 or f32");
  if (!q || !k_ext || !v_ext || !out || !qo_indptr || !kv_indptr)
    return fail(AKV_EINVAL, "akv_context_attention: null device pointer");
  // prefix keys are read from the pools through kv_indices
  if (kv_indices && (!k_buffer || !v_buffer))
    return fail(AKV_EINVAL, "akv_context_attention: prefix indices given without K/V pools");
  if ((q_positions == nullptr) != (kv_positions == nullptr))
    return fail(AKV_EINVAL, "akv_context_attention: needs both query and KV positions or neither");
  const int64_t strides[] = {q_stride_t,    q_stride_h,    k_ext_stride_t, k_ext_stride_h, v_ext_stride_t,
                             v_ext_stride_h, k_stride_slot, k_stride_head,  v_stride_slot,  v_stride_head,
                             out_stride_t,  out_stride_h};
  for (int64_t s : strides) {
    if (s % 8 != 0) return fail(AKV_EINVAL, "akv_context_attention: row strides must be multiples of 8 elements");
    if (s < 0 || s > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_context_attention: strides must fit 31 bits");
  }
  const uintptr_t bases = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_ext) |
                          reinterpret_cast<uintptr_t>(v_ext) | reinterpret_cast<uintptr_t>(k_buffer) |
                          reinterpret_cast<uintptr_t>(v_buffer) | reinterpret_cast<uintptr_t>(out);
  if (bases & 15) return fail(AKV_EINVAL, "akv_context_attention: tensors must be 16-byte aligned");
  if (n_segments > 65535 || kv_heads > 65535)
    return fail(AKV_EINVAL, "akv_context_attention: batch too large");
  // masked scores are -inf before the scale: the softmax needs scale > 0
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(AKV_EINVAL, "akv_context_attention: scale must be positive and finite");
  CtxArgs a{};
  a.q = static_cast<const __bf16*>(q);
  a.k_ext = static_cast<const __bf16*>(k_ext);
  a.v_ext = static_cast<const __bf16*>(v_ext);
  a.k_pool = static_cast<const __bf16*>(k_buffer);
  a.v_pool = static_cast<const __bf16*>(v_buffer);
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.q_pos = q_positions;
  a.kv_pos = kv_positions;
  a.sinks = sinks;
  a.out = out;
  a.q_st = static_cast<int32_t>(q_stride_t);
  a.q_sh = static_cast<int32_t>(q_stride_h);
  a.ke_st = static_cast<int32_t>(k_ext_stride_t);
  a.ke_sh = static_cast<int32_t>(k_ext_stride_h);
  a.ve_st = static_cast<int32_t>(v_ext_stride_t);
  a.ve_sh = static_cast<int32_t>(v_ext_stride_h);
  a.kp_ss = static_cast<int32_t>(k_stride_slot);
  a.kp_sh = static_cast<int32_t>(k_stride_head);
  a.vp_ss = static_cast<int32_t>(v_stride_slot);
  a.vp_sh = static_cast<int32_t>(v_stride_head);
  a.o_st = static_cast<int32_t>(out_stride_t);
  a.o_sh = static_cast<int32_t>(out_stride_h);
  a.indptr_i64 = indptr_dtype == AKV_I64;
  // as the extend kernel this replaces, a window applies only when it is
  // positive (akv/system/sglang.patch:527-541): 0 means plain causal
  a.window = sliding_window > 0 ? sliding_window : -1;
  a.scale_log2 = scale * kLog2e;
  a.out_f32 = out_dtype == AKV_F32;
  a.group = q_heads / kv_heads;
  while ((1 << a.group_shift) < a.group) ++a.group_shift;  // rows per token: the group padded to 2^shift
  const int tile_dim = head_dim > 64 ? 128 : 64;
  a.tokens_per_block = rows_per_block(tile_dim) >> a.group_shift;
  a.head_dim = head_dim;
  a.cap = logit_cap;
  a.cap_log2 = logit_cap * kLog2e;
  const int64_t blocks = (max_query_len + a.tokens_per_block - 1) / a.tokens_per_block;
  if (blocks * kv_heads > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_context_attention: queries too long");
  a.kv_heads = kv_heads;
  const dim3 grid(static_cast<unsigned>(blocks * kv_heads), 1u, static_cast<unsigned>(n_segments));
  hipStream_t st = as_stream(stream);
  const bool idx64 = indices_dtype == AKV_I64;
  const int pos = q_positions == nullptr ? 0 : (positions_dtype == AKV_I64 ? 2 : 1);
  launch_typed(head_dim, idx64, pos, grid, st, a);
  return check_launch("akv_context_attention");
}
