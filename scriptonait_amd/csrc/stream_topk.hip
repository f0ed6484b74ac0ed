// The streaming top-k kernel (stream_row.h) and its launch: top-k rows of
// vocabularies past the register path, one persistent workgroup per CU.
#include <algorithm>

#include "stream_row.h"

namespace llmhip {

template <bool VEC>
__global__ __launch_bounds__(kBlock) void sample_stream_kernel(SampleArgs a) {
  __shared__ StreamKernelLds L;
  stream_rows<VEC>(a, L);
}

// vec: rows 16-byte aligned with a stride of a multiple of 4 floats.
hipError_t launch_stream(const SampleArgs& a0, bool vec, hipStream_t s) {
  SampleArgs a = a0;
  a.launch_rows = launch_grid(a);
  if (a.launch_rows == 0) return hipSuccess;
  const uint32_t grid = std::min(a.launch_rows, std::max(a.cus, 1u));
  if (vec) {
    hipLaunchKernelGGL(sample_stream_kernel<true>, dim3(grid), dim3(kBlock), 0, s, a);
  } else {
    hipLaunchKernelGGL(sample_stream_kernel<false>, dim3(grid), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace llmhip
