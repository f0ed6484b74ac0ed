// The register-path kernels for V <= 16384 (one, two or four float4 chunks
// per thread), calls without a count table.
#include "fast_kernel.h"

namespace llmhip {
template hipError_t launch_fast_nch<1, false>(const SampleArgs&, bool, bool, hipStream_t);
template hipError_t launch_fast_nch<2, false>(const SampleArgs&, bool, bool, hipStream_t);
template hipError_t launch_fast_nch<4, false>(const SampleArgs&, bool, bool, hipStream_t);
}  // namespace llmhip
