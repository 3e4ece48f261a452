// Shared helpers of the akv_amd HIP library (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include "abi_common.h"

namespace akv {

// Maps the state after a kernel launch to AKV_OK / AKV_EHIP.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool valid_index_dtype(int32_t d) { return d == AKV_I32 || d == AKV_I64; }

// A consumer's gate: true when the compaction status word it was given says
// the lists must not be used.  Every workgroup reads the word (one load,
// issued with its first index loads) and stops before it dereferences a
// list entry or stores anything.
__device__ __forceinline__ bool gated(const int32_t* status) {
  return status && (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & AKV_STATUS_UNUSABLE) != 0;
}

// Reads element i of an int32 or int64 device vector as int64.  `is64` is
// uniform across the grid, so the branch never diverges.
__device__ __forceinline__ int64_t load_index(const void* p, bool is64, int64_t i) {
  return is64 ? static_cast<const int64_t*>(p)[i]
              : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

__device__ __forceinline__ void store_index(void* p, bool is64, int64_t i, int64_t v) {
  if (is64)
    static_cast<int64_t*>(p)[i] = v;
  else
    static_cast<int32_t*>(p)[i] = static_cast<int32_t>(v);
}

}  // namespace akv
