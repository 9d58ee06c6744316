// Shared device/host helpers for the gfx950 flash-mlm kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flash_mlm_hip.h"

#define FMLM_DEV __device__ __forceinline__

namespace fmlm {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

inline int elem_size(int dtype) {
  switch (dtype) {
    case FMLM_DTYPE_BF16:
    case FMLM_DTYPE_F16:
      return 2;
    case FMLM_DTYPE_F32:
      return 4;
    default:
      return 0;
  }
}

// Start of sequence b in packed token space.
FMLM_DEV int seq_start(const int32_t* cu, int b, int N) { return cu ? cu[b] : b * N; }

// Index of the sequence whose packed token range [cu[s], cu[s+1]) holds token j
// (cu non-decreasing, 0 <= j < cu[B]).  Empty sequences are skipped because
// the search returns the last s with cu[s] <= j.
FMLM_DEV int find_seq(const int32_t* cu, int B, int j) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= j)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

}  // namespace fmlm
