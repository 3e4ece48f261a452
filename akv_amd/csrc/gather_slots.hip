// Batched owner-row -> slot gather (gfx950): the device half of a batch's
// ownership advance, publication, Drop of borrowed owners and terminal
// table reads.
//
// Each request b exposes a virtual slot vector made of up to three device
// pieces, src0 ++ src1 ++ src2 (for an advance: its previous owners, this
// forward's birth slots and its fresh slots).  The host planner emits, per
// request, segments of owner-row indices into that vector (occurrence
// slots, copy sources, copy destinations, successor owners, retired pages,
// SWA-released pages ...).  One launch resolves every segment of the batch:
// element i of the concatenation gets slot(b, rows[i]), or -1 for row -1
// (and for a row or request id out of range: no read outside the pieces).
// Elements [0, wide_count) go to `out_wide` (the slot dtype), the rest to
// `out_narrow` (int32: the copy lists the Reposition reads).
//
// Replaces, per request, a torch.cat of the three pieces plus one indexing
// launch per list (akv/system/sglang/srt/context_system/occurrence.py:
// 733-755, 757-767, 795-798, 856-864) and the batch concatenations of
// akv/system/sglang.patch:3174-3180.
#include "common.h"

namespace akv {
namespace {

constexpr int kThreads = 256;

struct GatherArgs {
  const int64_t* sources;  // [B][6]: ptr0, len0, ptr1, len1, ptr2, len2
  const int64_t* segment_offsets;  // [S + 1]
  const int64_t* segment_requests;  // [S]
  const int64_t* rows;  // [total]
  int64_t n_requests;
  int64_t n_segments;
  int64_t total;
  int64_t wide_count;
  void* out_wide;
  int32_t* out_narrow;
};

template <typename Slot>
__global__ void __launch_bounds__(kThreads) gather_slots_kernel(const GatherArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= a.total) return;
  // segment of element i: last s with offsets[s] <= i
  int64_t lo = 0, hi = a.n_segments;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (a.segment_offsets[mid] <= i)
      lo = mid;
    else
      hi = mid;
  }
  const int64_t b = a.segment_requests[lo];
  int64_t row = a.rows[i];
  int64_t v = -1;
  if (row >= 0 && b >= 0 && b < a.n_requests) {
    const int64_t* src = a.sources + 6 * b;
#pragma unroll
    for (int piece = 0; piece < 3; ++piece) {
      const int64_t len = src[2 * piece + 1];
      if (row < len) {
        v = static_cast<int64_t>(reinterpret_cast<const Slot*>(src[2 * piece])[row]);
        break;
      }
      row -= len;
    }
  }
  if (i < a.wide_count)
    static_cast<Slot*>(a.out_wide)[i] = static_cast<Slot>(v);
  else
    a.out_narrow[i - a.wide_count] = static_cast<int32_t>(v);
}

}  // namespace
}  // namespace akv

extern "C" int akv_gather_slots(int32_t slot_dtype, const int64_t* sources, int64_t n_requests, int64_t n_segments,
                                const int64_t* segment_offsets, const int64_t* segment_requests,
                                const int64_t* rows, int64_t total, int64_t wide_count, void* out_wide,
                                int32_t* out_narrow, void* stream) {
  using namespace akv;
  if (!valid_index_dtype(slot_dtype)) return fail(AKV_EINVAL, "akv_gather_slots: slot dtype must be int32 or int64");
  if (total < 0 || n_requests < 0 || n_segments < 0 || wide_count < 0 || wide_count > total)
    return fail(AKV_EINVAL, "akv_gather_slots: invalid sizes");
  if (total == 0) return AKV_OK;
  if (n_requests == 0 || n_segments == 0 || !sources || !segment_offsets || !segment_requests || !rows ||
      (wide_count && !out_wide) || (wide_count < total && !out_narrow))
    return fail(AKV_EINVAL, "akv_gather_slots: null pointer");
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_gather_slots: too many elements");
  GatherArgs a{sources, segment_offsets, segment_requests, rows, n_requests, n_segments, total, wide_count, out_wide,
               out_narrow};
  if (slot_dtype == AKV_I64)
    hipLaunchKernelGGL(gather_slots_kernel<int64_t>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       as_stream(stream), a);
  else
    hipLaunchKernelGGL(gather_slots_kernel<int32_t>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       as_stream(stream), a);
  return check_launch("akv_gather_slots");
}
