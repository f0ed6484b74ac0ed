// The register-path kernels for decode steps with a count table
// (llmhip_decode_step_counts): the same kernel as the other calls, compiled
// with the table's reads and updates in place of the history walk.
#include "fast_kernel.h"

namespace llmhip {

hipError_t launch_fast_counts(const SampleArgs& a, bool vec, bool bigk, hipStream_t s) {
  return launch_fast_mode<true>(a, vec, bigk, s);
}

}  // namespace llmhip
