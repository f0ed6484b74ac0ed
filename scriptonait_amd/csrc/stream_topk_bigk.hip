// The streaming top-k kernels for launches with some row of K > 64.
#include "stream_kernel.h"

namespace llmhip {

template hipError_t launch_stream_k<true>(const SampleArgs&, bool, hipStream_t);

}  // namespace llmhip
