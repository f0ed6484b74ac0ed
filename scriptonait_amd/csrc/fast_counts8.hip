// The register-path kernels for decode steps with a count table, 16384 < V
// <= 32768.
#include "fast_kernel.h"

namespace llmhip {
template hipError_t launch_fast_nch<8, true>(const SampleArgs&, bool, bool, hipStream_t);
}  // namespace llmhip
