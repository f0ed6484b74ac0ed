// The register-path kernels for decode steps with a count table, V <= 16384.
#include "fast_kernel.h"

namespace llmhip {
template hipError_t launch_fast_nch<1, true>(const SampleArgs&, bool, bool, hipStream_t);
template hipError_t launch_fast_nch<2, true>(const SampleArgs&, bool, bool, hipStream_t);
template hipError_t launch_fast_nch<4, true>(const SampleArgs&, bool, bool, hipStream_t);
}  // namespace llmhip
