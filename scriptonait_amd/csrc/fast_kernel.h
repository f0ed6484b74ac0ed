// The register-path kernel and its launch, templated on count-table mode:
// decode steps with a count table run their own instantiations (compiled
// in fast_counts.hip), so the other calls carry none of that code.
#pragma once
#include "fast_row.h"
#include "general_row.h"
#include "sampler_common.h"

namespace llmhip {

static_assert(kMaxFastK <= kSelCap, "hand-overs select in LDS");

template <int NCH, bool VEC, bool GREEDY, bool CMODE, bool BIGK>
__global__ __launch_bounds__(kBlock) void sample_fast_kernel(SampleArgs a) {
  __shared__ FastLds<NCH, BIGK> L;
  if (__builtin_expect(!fast_row<NCH, VEC, GREEDY, CMODE, BIGK>(a, L), 0)) {
    if (threadIdx.x == 0) atomicAdd(a.handovers, 1u);
    __syncthreads();
    general_row<false>(a, launch_row(a), L.gen, true);  // greedy or K <= kMaxFastK: no whole-row sort
  }
}

// One launch per row class present: greedy rows and top-k rows run in
// kernels compiled apart, so neither carries the other's registers. bigk:
// some top-k row has K > 64.
template <int NCH, bool CMODE>
hipError_t launch_fast_nch(const SampleArgs& a0, bool vec, bool bigk, hipStream_t s) {
  SampleArgs a = a0;
  uint32_t grid;
  a.row_class_mask = kClassGreedy;
  if ((a0.row_class_mask & kClassGreedy) && (grid = launch_grid(a)) != 0u) {
    if (vec) {
      hipLaunchKernelGGL((sample_fast_kernel<NCH, true, true, CMODE, false>), dim3(grid), dim3(kBlock), 0, s, a);
    } else {
      hipLaunchKernelGGL((sample_fast_kernel<NCH, false, true, CMODE, false>), dim3(grid), dim3(kBlock), 0, s, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  a.row_class_mask = kClassTopK;
  if ((a0.row_class_mask & kClassTopK) && (grid = launch_grid(a)) != 0u) {
    if (vec && bigk) {
      hipLaunchKernelGGL((sample_fast_kernel<NCH, true, false, CMODE, true>), dim3(grid), dim3(kBlock), 0, s, a);
    } else if (vec) {
      hipLaunchKernelGGL((sample_fast_kernel<NCH, true, false, CMODE, false>), dim3(grid), dim3(kBlock), 0, s, a);
    } else if (bigk) {
      hipLaunchKernelGGL((sample_fast_kernel<NCH, false, false, CMODE, true>), dim3(grid), dim3(kBlock), 0, s, a);
    } else {
      hipLaunchKernelGGL((sample_fast_kernel<NCH, false, false, CMODE, false>), dim3(grid), dim3(kBlock), 0, s, a);
    }
  }
  return hipGetLastError();
}

// Each (NCH, CMODE) instantiation is compiled in a file of its own
// (fast_nch8.hip, fast_nch_small.hip, fast_counts8.hip,
// fast_counts_small.hip), so the library's kernels build in parallel.
extern template hipError_t launch_fast_nch<1, false>(const SampleArgs&, bool, bool, hipStream_t);
extern template hipError_t launch_fast_nch<2, false>(const SampleArgs&, bool, bool, hipStream_t);
extern template hipError_t launch_fast_nch<4, false>(const SampleArgs&, bool, bool, hipStream_t);
extern template hipError_t launch_fast_nch<8, false>(const SampleArgs&, bool, bool, hipStream_t);
extern template hipError_t launch_fast_nch<1, true>(const SampleArgs&, bool, bool, hipStream_t);
extern template hipError_t launch_fast_nch<2, true>(const SampleArgs&, bool, bool, hipStream_t);
extern template hipError_t launch_fast_nch<4, true>(const SampleArgs&, bool, bool, hipStream_t);
extern template hipError_t launch_fast_nch<8, true>(const SampleArgs&, bool, bool, hipStream_t);

template <bool CMODE>
hipError_t launch_fast_mode(const SampleArgs& a, bool vec, bool bigk, hipStream_t s) {
  switch (fast_nch(a.V)) {
    case 1: return launch_fast_nch<1, CMODE>(a, vec, bigk, s);
    case 2: return launch_fast_nch<2, CMODE>(a, vec, bigk, s);
    case 4: return launch_fast_nch<4, CMODE>(a, vec, bigk, s);
    default: return launch_fast_nch<8, CMODE>(a, vec, bigk, s);
  }
}

}  // namespace llmhip
