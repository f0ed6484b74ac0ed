// The streaming top-k kernels without the large-K rank and tail, and the
// launch that picks between those and stream_topk_bigk.hip's.
#include "stream_kernel.h"

namespace llmhip {

template hipError_t launch_stream_k<false>(const SampleArgs&, bool, hipStream_t);

// bigk: some row of the launch has K > 64.
hipError_t launch_stream(const SampleArgs& a, bool vec, bool bigk, hipStream_t s) {
  return bigk ? launch_stream_k<true>(a, vec, s) : launch_stream_k<false>(a, vec, s);
}

}  // namespace llmhip
