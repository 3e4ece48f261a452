// Decode metadata over compacted request rows (gfx950).
//
//   akv_decode_indices   context_decode_indices
//                        (akv/system/sglang/kernels/ops/attention/context_page_table.py:34-76)
//   akv_window_lengths   context_window_lengths (context_page_table.py:7-31)
//   akv_build_indptr     kv_indptr[1:] = cumsum(seq_lens) (akv/system/sglang.patch:2266-2268)
//   akv_write_row_slots  write_row_slots (akv/system/sglang/kernels/ops/memory/context_rows.py:7-15)
//   akv_write_extend_rows write_req_to_token_pool_triton with RowPointers
//                        (akv/system/sglang.patch:238-278, caller sglang.patch:4066-4090)
//
// The reference walks each request with one program in 256-token steps; here
// every request gets several workgroups that stride over its range, so one
// long request no longer serialises the whole launch.  Registry rows are
// int64[6] = (raw_ids_ptr, positions_ptr, prompt_len, active, next_pos,
// row_ptr); a zero raw_ids_ptr marks an ordinary request.
#include "common.h"

extern "C" __device__ long long __ockl_wfred_add_i64(long long);

namespace akv {
namespace {

// workgroups per request, and independent gathers each thread keeps in flight
// (one row entry costs two dependent loads: raw id, then slot)
constexpr int kBlocksPerRequest = 16;
constexpr int kUnroll = 4;

struct DecodeArgs {
  const int64_t* registry;
  const int32_t* table;
  int64_t row_stride;
  const void* rows;
  const void* lengths;
  const void* indptr;
  void* output;
  const void* starts;
  const void* mapping;
  const int32_t* gate;  // compaction status word, or nullptr
  int64_t multiplier;
  int32_t n_requests;
  bool rows64, lengths64, indptr64, output64, starts64, mapping64;
};

__global__ void __launch_bounds__(256) decode_indices_kernel(const DecodeArgs a) {
  const int b = blockIdx.y;
  const int64_t row = load_index(a.rows, a.rows64, b);
  const int64_t length = load_index(a.lengths, a.lengths64, b);
  const int64_t offset = load_index(a.indptr, a.indptr64, b);
  const int64_t start = a.starts ? load_index(a.starts, a.starts64, b) : 0;
  const int64_t* entry = a.registry + row * 6;
  const int64_t pointer = entry[0];
  // the reference narrows prompt/active to int32 before use
  const int32_t prompt = static_cast<int32_t>(entry[2]);
  const int32_t active = static_cast<int32_t>(entry[3]);
  const int32_t* raw_ids = reinterpret_cast<const int32_t*>(pointer);
  const int64_t row_pointer = entry[5];
  const int32_t* raw_row = row_pointer != 0 ? reinterpret_cast<const int32_t*>(row_pointer)
                                            : a.table + row * a.row_stride;
  // a closed gate stops the request before its raw ids and row entries
  if (gated(a.gate)) return;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  auto raw_of = [&](int64_t i) -> int64_t {
    const int64_t logical = start + i;
    if (pointer == 0) return logical;
    return logical < active ? raw_ids[logical] : prompt + logical - active;
  };
  auto emit = [&](int64_t i, int64_t slot) {
    if (a.mapping) slot = load_index(a.mapping, a.mapping64, slot) * a.multiplier;
    store_index(a.output, a.output64, offset + i, slot);
  };
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i + (kUnroll - 1) * step < length; i += kUnroll * step) {
    int64_t raw[kUnroll], slot[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) raw[u] = raw_of(i + u * step);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) slot[u] = raw_row[raw[u]];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) emit(i + u * step, slot[u]);
  }
  for (; i < length; i += step) emit(i, raw_row[raw_of(i)]);
}

struct WindowArgs {
  const int64_t* registry;
  const void* rows;
  const void* lengths;
  void* output;
  void* starts;
  int64_t window;
  int32_t n_requests;
  bool rows64, lengths64, output64;
};

__global__ void __launch_bounds__(256) window_lengths_kernel(const WindowArgs a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.n_requests) return;
  const int64_t row = load_index(a.rows, a.rows64, b);
  const int64_t length = load_index(a.lengths, a.lengths64, b);
  const int64_t* entry = a.registry + row * 6;
  int64_t result = length < a.window ? length : a.window;
  if (entry[0] != 0) {
    const int32_t* positions = reinterpret_cast<const int32_t*>(entry[1]);
    const int32_t active = static_cast<int32_t>(entry[3]);
    const int32_t next_pos = static_cast<int32_t>(entry[4]);
    const int64_t generated = length - active;
    // visible keys satisfy q_pos - k_pos <= window (inclusive)
    const int64_t lower = next_pos + generated - 1 - a.window;
    int32_t lo = 0, hi = active;
    while (lo < hi) {
      const int32_t mid = lo + ((hi - lo) >> 1);
      if (positions[mid] < lower)
        lo = mid + 1;
      else
        hi = mid;
    }
    const int64_t skipped = lower - next_pos > 0 ? lower - next_pos : 0;
    result = active - lo + generated - skipped;
  }
  store_index(a.output, a.output64, b, result);
  if (a.starts) store_index(a.starts, a.lengths64, b, length - result);
}

struct IndptrArgs {
  const void* lengths;
  void* indptr;
  int32_t* last_page_len;
  int64_t scale;
  int32_t n_requests;
  int32_t page_size;
  bool lengths64, indptr64;
};

// One workgroup: exclusive scan of the request lengths.
__global__ void __launch_bounds__(1024) build_indptr_kernel(const IndptrArgs a) {
  __shared__ int64_t wave_tot[16];
  __shared__ int64_t carry;
  if (a.scale != 1) {
    for (int b = threadIdx.x; b <= a.n_requests; b += blockDim.x)
      store_index(a.indptr, a.indptr64, b, static_cast<int64_t>(b) * a.scale);
    return;
  }
  if (threadIdx.x == 0) {
    carry = 0;
    store_index(a.indptr, a.indptr64, 0, 0);
  }
  __syncthreads();
  const int lane = __lane_id();
  const int w = threadIdx.x >> 6;
  for (int base = 0; base < a.n_requests; base += blockDim.x) {
    const int b = base + threadIdx.x;
    const int64_t len = b < a.n_requests ? load_index(a.lengths, a.lengths64, b) : 0;
    int64_t inc = len;
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t up = __shfl_up(inc, off);
      if (lane >= off) inc += up;
    }
    if (lane == 63) wave_tot[w] = inc;
    __syncthreads();
    int64_t prefix = carry;
    for (int q = 0; q < w; ++q) prefix += wave_tot[q];
    if (b < a.n_requests) {
      store_index(a.indptr, a.indptr64, b + 1, prefix + inc);
      if (a.last_page_len) a.last_page_len[b] = len > 0 ? static_cast<int32_t>((len - 1) % a.page_size + 1) : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int q = 0; q < (int)((blockDim.x + 63) / 64); ++q) carry += wave_tot[q];
    }
    __syncthreads();
  }
}

struct RowSlotArgs {
  const int64_t* pointers;
  const void* rows;
  const void* columns;
  const void* values;
  int64_t n;
  bool rows64, columns64, values64;
};

__global__ void __launch_bounds__(256) write_row_slots_kernel(const RowSlotArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  const int64_t row = load_index(a.rows, a.rows64, i);
  const int64_t column = load_index(a.columns, a.columns64, i);
  int32_t* p = reinterpret_cast<int32_t*>(a.pointers[row]);
  p[column] = static_cast<int32_t>(load_index(a.values, a.values64, i));
}

// Extend write: per request b, row[0, pre) = prefix_b[0, pre) and
// row[pre, seq) = out_cache_loc[start_b + (0 .. seq - pre)), start_b the
// exclusive prefix of extend_lens.  Grid (kExtendSlices, B): each workgroup
// writes one slice of its request's row.
constexpr int kExtendSlices = 8;

struct ExtendArgs {
  int32_t* table;
  int64_t row_stride;
  const int64_t* row_pointers;
  const void* req_rows;
  const int64_t* prefix_ptrs;
  const void* pre_lens;
  const void* seq_lens;
  const void* extend_lens;
  const void* out_cache_loc;
  bool rows64, prefix64, lens64, loc64;
};

__global__ void __launch_bounds__(256) write_extend_rows_kernel(const ExtendArgs a) {
  const int b = blockIdx.y;
  // start of this request's new slots: sum of the earlier extend lengths
  int64_t before = 0;
  for (int i = threadIdx.x; i < b; i += 256) before += load_index(a.extend_lens, a.lens64, i);
  before = __ockl_wfred_add_i64(before);
  __shared__ int64_t part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = before;
  __syncthreads();
  const int64_t start = part[0] + part[1] + part[2] + part[3];
  const int64_t r = load_index(a.req_rows, a.rows64, b);
  int32_t* row = a.row_pointers ? reinterpret_cast<int32_t*>(a.row_pointers[r]) : a.table + r * a.row_stride;
  const int64_t pre = load_index(a.pre_lens, a.lens64, b);
  const int64_t seq = load_index(a.seq_lens, a.lens64, b);
  const void* prefix = reinterpret_cast<const void*>(a.prefix_ptrs[b]);
  const int64_t slice = ((seq + kExtendSlices - 1) / kExtendSlices + 255) / 256 * 256;
  const int64_t lo = blockIdx.x * slice;
  const int64_t hi = lo + slice < seq ? lo + slice : seq;
  for (int64_t j = lo + threadIdx.x; j < hi; j += 256) {
    const int64_t v = j < pre ? load_index(prefix, a.prefix64, j) : load_index(a.out_cache_loc, a.loc64, start + j - pre);
    row[j] = static_cast<int32_t>(v);
  }
}

}  // namespace
}  // namespace akv

extern "C" int akv_decode_indices(const int64_t* registry, const int32_t* table, int64_t row_stride,
                                  const void* rows, int32_t rows_dtype, const void* lengths,
                                  int32_t lengths_dtype, const void* indptr, int32_t indptr_dtype,
                                  void* output, int32_t output_dtype, const void* starts,
                                  int32_t starts_dtype, const void* mapping, int32_t mapping_dtype,
                                  int64_t multiplier, int32_t n_requests, const int32_t* status,
                                  void* stream) {
  using namespace akv;
  if (n_requests < 0) return fail(AKV_EINVAL, "akv_decode_indices: negative batch size");
  if (n_requests == 0) return AKV_OK;
  if (n_requests > 65535) return fail(AKV_EINVAL, "akv_decode_indices: batch of %d requests exceeds one launch", n_requests);
  if (!registry || !table || !rows || !lengths || !indptr || !output)
    return fail(AKV_EINVAL, "akv_decode_indices: null device pointer");
  if (!valid_index_dtype(rows_dtype) || !valid_index_dtype(lengths_dtype) || !valid_index_dtype(indptr_dtype) ||
      !valid_index_dtype(output_dtype) || (starts && !valid_index_dtype(starts_dtype)) ||
      (mapping && !valid_index_dtype(mapping_dtype)))
    return fail(AKV_EINVAL, "akv_decode_indices: index vectors must be int32 or int64");
  DecodeArgs a{};
  a.registry = registry;
  a.table = table;
  a.row_stride = row_stride;
  a.rows = rows;
  a.lengths = lengths;
  a.indptr = indptr;
  a.output = output;
  a.starts = starts;
  a.mapping = mapping;
  a.gate = status;
  a.multiplier = multiplier;
  a.n_requests = n_requests;
  a.rows64 = rows_dtype == AKV_I64;
  a.lengths64 = lengths_dtype == AKV_I64;
  a.indptr64 = indptr_dtype == AKV_I64;
  a.output64 = output_dtype == AKV_I64;
  a.starts64 = starts_dtype == AKV_I64;
  a.mapping64 = mapping_dtype == AKV_I64;
  hipLaunchKernelGGL(decode_indices_kernel, dim3(kBlocksPerRequest, n_requests), dim3(256), 0,
                     as_stream(stream), a);
  return check_launch("akv_decode_indices");
}

extern "C" int akv_window_lengths(const int64_t* registry, const void* rows, int32_t rows_dtype,
                                  const void* lengths, int32_t lengths_dtype, void* output,
                                  int32_t output_dtype, void* starts, int64_t window,
                                  int32_t n_requests, void* stream) {
  using namespace akv;
  if (n_requests < 0) return fail(AKV_EINVAL, "akv_window_lengths: negative batch size");
  if (n_requests == 0) return AKV_OK;
  if (!registry || !rows || !lengths || !output) return fail(AKV_EINVAL, "akv_window_lengths: null device pointer");
  if (!valid_index_dtype(rows_dtype) || !valid_index_dtype(lengths_dtype) || !valid_index_dtype(output_dtype))
    return fail(AKV_EINVAL, "akv_window_lengths: index vectors must be int32 or int64");
  WindowArgs a{};
  a.registry = registry;
  a.rows = rows;
  a.lengths = lengths;
  a.output = output;
  a.starts = starts;
  a.window = window;
  a.n_requests = n_requests;
  a.rows64 = rows_dtype == AKV_I64;
  a.lengths64 = lengths_dtype == AKV_I64;
  a.output64 = output_dtype == AKV_I64;
  hipLaunchKernelGGL(window_lengths_kernel, dim3((n_requests + 255) / 256), dim3(256), 0, as_stream(stream), a);
  return check_launch("akv_window_lengths");
}

extern "C" int akv_build_indptr(const void* lengths, int32_t lengths_dtype, int32_t n_requests, void* indptr,
                                int32_t indptr_dtype, int32_t* last_page_len, int32_t page_size,
                                int64_t indptr_scale, void* stream) {
  using namespace akv;
  if (n_requests < 0) return fail(AKV_EINVAL, "akv_build_indptr: negative batch size");
  if (!indptr) return fail(AKV_EINVAL, "akv_build_indptr: null indptr");
  if (indptr_scale == 1 && n_requests > 0 && !lengths) return fail(AKV_EINVAL, "akv_build_indptr: null lengths");
  if (page_size <= 0) return fail(AKV_EINVAL, "akv_build_indptr: page_size must be positive");
  if (!valid_index_dtype(indptr_dtype) || (lengths && !valid_index_dtype(lengths_dtype)))
    return fail(AKV_EINVAL, "akv_build_indptr: index vectors must be int32 or int64");
  IndptrArgs a{};
  a.lengths = lengths;
  a.indptr = indptr;
  a.last_page_len = last_page_len;
  a.scale = indptr_scale;
  a.n_requests = n_requests;
  a.page_size = page_size;
  a.lengths64 = lengths_dtype == AKV_I64;
  a.indptr64 = indptr_dtype == AKV_I64;
  hipLaunchKernelGGL(build_indptr_kernel, dim3(1), dim3(1024), 0, as_stream(stream), a);
  return check_launch("akv_build_indptr");
}

extern "C" int akv_write_row_slots(const int64_t* pointers, const void* rows, int32_t rows_dtype,
                                   const void* columns, int32_t columns_dtype, const void* values,
                                   int32_t values_dtype, int64_t n, void* stream) {
  using namespace akv;
  if (n < 0) return fail(AKV_EINVAL, "akv_write_row_slots: negative count");
  if (n == 0) return AKV_OK;
  if (!pointers || !rows || !columns || !values) return fail(AKV_EINVAL, "akv_write_row_slots: null device pointer");
  if (!valid_index_dtype(rows_dtype) || !valid_index_dtype(columns_dtype) || !valid_index_dtype(values_dtype))
    return fail(AKV_EINVAL, "akv_write_row_slots: index vectors must be int32 or int64");
  RowSlotArgs a{};
  a.pointers = pointers;
  a.rows = rows;
  a.columns = columns;
  a.values = values;
  a.n = n;
  a.rows64 = rows_dtype == AKV_I64;
  a.columns64 = columns_dtype == AKV_I64;
  a.values64 = values_dtype == AKV_I64;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(AKV_EINVAL, "akv_write_row_slots: too many entries");
  hipLaunchKernelGGL(write_row_slots_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream), a);
  return check_launch("akv_write_row_slots");
}

extern "C" int akv_write_extend_rows(int32_t* table, int64_t row_stride, const int64_t* row_pointers,
                                     const void* req_rows, int32_t rows_dtype, const int64_t* prefix_ptrs,
                                     int32_t prefix_dtype, const void* pre_lens, const void* seq_lens,
                                     const void* extend_lens, int32_t lens_dtype, const void* out_cache_loc,
                                     int32_t loc_dtype, int32_t n_requests, void* stream) {
  using namespace akv;
  if (n_requests < 0) return fail(AKV_EINVAL, "akv_write_extend_rows: negative batch size");
  if (n_requests == 0) return AKV_OK;
  if (n_requests > 65535)
    return fail(AKV_EINVAL, "akv_write_extend_rows: batch of %d requests exceeds one launch", n_requests);
  if ((!table && !row_pointers) || !req_rows || !prefix_ptrs || !pre_lens || !seq_lens || !extend_lens ||
      !out_cache_loc)
    return fail(AKV_EINVAL, "akv_write_extend_rows: null device pointer");
  if (!valid_index_dtype(rows_dtype) || !valid_index_dtype(prefix_dtype) || !valid_index_dtype(lens_dtype) ||
      !valid_index_dtype(loc_dtype))
    return fail(AKV_EINVAL, "akv_write_extend_rows: index vectors must be int32 or int64");
  ExtendArgs a{};
  a.table = table;
  a.row_stride = row_stride;
  a.row_pointers = row_pointers;
  a.req_rows = req_rows;
  a.prefix_ptrs = prefix_ptrs;
  a.pre_lens = pre_lens;
  a.seq_lens = seq_lens;
  a.extend_lens = extend_lens;
  a.out_cache_loc = out_cache_loc;
  a.rows64 = rows_dtype == AKV_I64;
  a.prefix64 = prefix_dtype == AKV_I64;
  a.lens64 = lens_dtype == AKV_I64;
  a.loc64 = loc_dtype == AKV_I64;
  hipLaunchKernelGGL(write_extend_rows_kernel, dim3(kExtendSlices, static_cast<unsigned>(n_requests)), dim3(256), 0,
                     as_stream(stream), a);
  return check_launch("akv_write_extend_rows");
}
