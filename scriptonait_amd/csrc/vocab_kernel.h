// The full-vocabulary kernel (vocab_row.h) and its launch, templated on
// PLAIN (no allowed mask, no ring, no penalized row): each instantiation is
// compiled in a file of its own (vocab_full.hip, vocab_plain.hip).
#pragma once
#include "general_row.h"
#include "sampler_common.h"
#include "vocab_row.h"

namespace llmhip {

// Rows it cannot certify take the sorting path in the same workgroup.
template <bool PLAIN>
__global__ __launch_bounds__(kBlock) void sample_vocab_kernel(SampleArgs a) {
  __shared__ union {
    VocabLds v;
    GenLds gen;
  } L;
  const uint32_t b = launch_row(a);
  if (b >= a.B) return;
  if (!a.row_cls_on && !(route_class(load_params(a, b), a.V) & a.row_class_mask)) return;
  const bool vec4 = (reinterpret_cast<uintptr_t>(a.logits) % 16u == 0u) && (a.ld % 4u == 0u);
  if (!vocab_row<PLAIN>(a, b, L.v, vec4)) {
    if (threadIdx.x == 0) atomicAdd(a.handovers, 1u);
    __syncthreads();
    general_row(a, b, L.gen, true);
  }
  LLMHIP_MARK(11);
}

template <bool PLAIN>
hipError_t launch_vocab_k(const SampleArgs& a, hipStream_t s) {
  const uint32_t grid = launch_grid(a);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(sample_vocab_kernel<PLAIN>, dim3(grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

extern template hipError_t launch_vocab_k<false>(const SampleArgs&, hipStream_t);
extern template hipError_t launch_vocab_k<true>(const SampleArgs&, hipStream_t);

}  // namespace llmhip
