// The full-vocabulary kernel for calls without an allowed mask, a ring or a
// penalized row.
#include "vocab_kernel.h"

namespace llmhip {

template hipError_t launch_vocab_k<true>(const SampleArgs&, hipStream_t);

}  // namespace llmhip
