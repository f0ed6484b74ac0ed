// The register-path kernels for 16384 < V <= 32768 (eight float4 chunks per
// thread), calls without a count table.
#include "fast_kernel.h"

namespace llmhip {
template hipError_t launch_fast_nch<8, false>(const SampleArgs&, bool, bool, hipStream_t);
}  // namespace llmhip
