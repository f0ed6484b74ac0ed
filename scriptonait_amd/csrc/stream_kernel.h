// The streaming top-k kernel (stream_row.h) and its launch, templated on
// BIGK (some row has K > 64): each BIGK instantiation is compiled in a file
// of its own (stream_topk.hip, stream_topk_bigk.hip).
#pragma once
#include <algorithm>

#include "stream_row.h"

namespace llmhip {

template <bool VEC, bool FULL, bool BIGK>
__global__ __launch_bounds__(kBlock) void sample_stream_kernel(SampleArgs a) {
  __shared__ StreamKernelLds L;
  stream_rows<VEC, FULL, BIGK>(a, L);
}

// One persistent workgroup per CU (at most one per row). vec: rows 16-byte
// aligned with a stride of a multiple of 4 floats.
template <bool BIGK>
hipError_t launch_stream_k(const SampleArgs& a0, bool vec, hipStream_t s) {
  SampleArgs a = a0;
  a.launch_rows = launch_grid(a);
  if (a.launch_rows == 0) return hipSuccess;
  const uint32_t grid = std::min(a.launch_rows, std::max(a.cus, 1u));
  const bool full = a.allowed || a.allowed_bits || a.ring_cap;
  if (vec && full) {
    hipLaunchKernelGGL((sample_stream_kernel<true, true, BIGK>), dim3(grid), dim3(kBlock), 0, s, a);
  } else if (vec) {
    hipLaunchKernelGGL((sample_stream_kernel<true, false, BIGK>), dim3(grid), dim3(kBlock), 0, s, a);
  } else if (full) {
    hipLaunchKernelGGL((sample_stream_kernel<false, true, BIGK>), dim3(grid), dim3(kBlock), 0, s, a);
  } else {
    hipLaunchKernelGGL((sample_stream_kernel<false, false, BIGK>), dim3(grid), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

extern template hipError_t launch_stream_k<false>(const SampleArgs&, bool, hipStream_t);
extern template hipError_t launch_stream_k<true>(const SampleArgs&, bool, hipStream_t);

}  // namespace llmhip
