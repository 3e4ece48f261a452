// Page-granular Drop + Reposition with copy-on-write (gfx950).
//
// The reference supports only page_size = 1
// (akv/system/sglang/kernels/ops/attention/context_reposition.py:153-154);
// this is the paged extension.  A request's raw row holds page-aligned token
// slots (page * P + offset).  After Drop + Reposition its kept tokens have
// final positions 0 .. kept-1 (their rank) and are packed page-dense by rank:
//   p0 = first dropped raw token / P; logical pages < p0 keep their physical
//   pages (shared prefix pages stay shared); every kept token of rank
//   r >= p0 * P moves out of place to fresh_pages[r / P - p0] * P + r % P --
//   copy-on-write for pages other requests still reference, no read/write
//   hazard for private ones -- with copy pair (birth position, r), so tokens
//   whose position did not change are bit copies in the Reposition;
//   the request releases its old pages of logical index >= p0.
//
// Because final positions are ranks, every output index is a direct function
// of the token's rank and the per-request bases the host derives from the
// CPU layout: one launch, one thread per raw token, no scan.
#include "common.h"

namespace akv {
namespace {

struct PagedArgs {
  const int64_t* req_offsets;
  int32_t* table;
  int64_t row_stride;
  const int64_t* row_pointers;
  const int64_t* req_rows;
  const uint8_t* keep;
  const int32_t* birth;
  const int32_t* final_pos;
  const int32_t* birth_slots;
  // bases[k * (B + 1) + b]: k = 0 copy_from (p0 * P), 1 kept, 2 copies,
  // 3 fresh pages, 4 new page-table entries, 5 released pages
  const int64_t* bases;
  const int32_t* fresh_pages;
  int32_t* copy_src;
  int32_t* copy_dst;
  int32_t* copy_pairs;
  int32_t* released;
  int32_t* page_table;
  int32_t* raw_indices;
  int32_t* active_positions;
  int32_t n_requests;
  int32_t page_size;
};

__global__ void __launch_bounds__(256) compact_pages_kernel(const PagedArgs a) {
  const int b = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t base = a.req_offsets[b];
  const int64_t n = a.req_offsets[b + 1] - base;
  if (i >= n) return;
  const int64_t B1 = a.n_requests + 1;
  const int64_t* copy_from_v = a.bases;
  const int64_t* kept_v = a.bases + B1;
  const int64_t* copies_v = a.bases + 2 * B1;
  const int64_t* fresh_v = a.bases + 3 * B1;
  const int64_t* pages_v = a.bases + 4 * B1;
  const int64_t* released_v = a.bases + 5 * B1;
  const int P = a.page_size;
  const int64_t r0 = a.req_rows[b];
  int32_t* row = a.row_pointers ? reinterpret_cast<int32_t*>(a.row_pointers[r0]) : a.table + r0 * a.row_stride;
  const int32_t old = a.birth_slots ? a.birth_slots[base + i] : row[i];
  const int64_t copy_from = copy_from_v[b];

  if (i % P == 0 && i >= copy_from) {
    const int64_t at = released_v[b] + (i - copy_from) / P;
    if (at < released_v[b + 1]) a.released[at] = old / P;
  }
  if (!a.keep[base + i]) {
    row[i] = -1;
    return;
  }
  const int32_t r = a.final_pos[base + i];
  const int64_t k_at = kept_v[b] + r;
  if (r >= 0 && k_at < kept_v[b + 1]) {
    a.raw_indices[k_at] = static_cast<int32_t>(i);
    a.active_positions[k_at] = r;
  }
  int32_t terminal = old;
  if (r >= copy_from) {
    const int64_t c = r - copy_from;
    const int64_t f_at = fresh_v[b] + c / P;
    const int64_t c_at = copies_v[b] + c;
    if (f_at < fresh_v[b + 1] && c_at < copies_v[b + 1]) {
      terminal = a.fresh_pages[f_at] * P + static_cast<int32_t>(c % P);
      a.copy_src[c_at] = old;
      a.copy_dst[c_at] = terminal;
      a.copy_pairs[2 * c_at] = a.birth[base + i];
      a.copy_pairs[2 * c_at + 1] = r;
    } else {
      terminal = -1;  // inconsistent bases: never point at another request's page
    }
  }
  if (r % P == 0) {
    const int64_t p_at = pages_v[b] + r / P;
    if (r >= 0 && p_at < pages_v[b + 1]) a.page_table[p_at] = terminal >= 0 ? terminal / P : -1;
  }
  row[i] = terminal;
}

}  // namespace
}  // namespace akv

extern "C" int akv_compact_pages(int32_t n_requests, const int64_t* req_offsets, int64_t max_tokens,
                                 int32_t page_size, int32_t* table, int64_t row_stride,
                                 const int64_t* row_pointers, const int64_t* req_rows, const uint8_t* keep,
                                 const int32_t* birth_positions, const int32_t* final_positions,
                                 const int32_t* birth_slots, const int64_t* bases, const int32_t* fresh_pages,
                                 int32_t* copy_src, int32_t* copy_dst, int32_t* copy_pairs,
                                 int32_t* released_pages, int32_t* page_table, int32_t* raw_indices,
                                 int32_t* active_positions, void* stream) {
  using namespace akv;
  if (n_requests < 0 || max_tokens < 0) return fail(AKV_EINVAL, "akv_compact_pages: negative size");
  if (n_requests == 0 || max_tokens == 0) return AKV_OK;
  if (page_size <= 0) return fail(AKV_EINVAL, "akv_compact_pages: page_size must be positive");
  if (!req_offsets || !req_rows || !keep || !birth_positions || !final_positions || !bases || !copy_src ||
      !copy_dst || !copy_pairs || !released_pages || !page_table || !raw_indices || !active_positions)
    return fail(AKV_EINVAL, "akv_compact_pages: null device pointer");
  if (!row_pointers && !table) return fail(AKV_EINVAL, "akv_compact_pages: need a request table or row pointers");
  const int64_t blocks = (max_tokens + 255) / 256;
  if (blocks > 0x7fffffffLL || n_requests > 65535)
    return fail(AKV_EINVAL, "akv_compact_pages: batch too large");
  PagedArgs a{};
  a.req_offsets = req_offsets;
  a.table = table;
  a.row_stride = row_stride;
  a.row_pointers = row_pointers;
  a.req_rows = req_rows;
  a.keep = keep;
  a.birth = birth_positions;
  a.final_pos = final_positions;
  a.birth_slots = birth_slots;
  a.bases = bases;
  a.fresh_pages = fresh_pages;
  a.copy_src = copy_src;
  a.copy_dst = copy_dst;
  a.copy_pairs = copy_pairs;
  a.released = released_pages;
  a.page_table = page_table;
  a.raw_indices = raw_indices;
  a.active_positions = active_positions;
  a.n_requests = n_requests;
  a.page_size = page_size;
  hipLaunchKernelGGL(compact_pages_kernel, dim3(static_cast<unsigned>(blocks), n_requests), dim3(256), 0,
                     as_stream(stream), a);
  return check_launch("akv_compact_pages");
}
