// The full-vocabulary kernel for calls with an allowed mask, a ring or a
// penalized row, and the launch that picks between it and vocab_plain.hip's.
#include "vocab_kernel.h"

namespace llmhip {

template hipError_t launch_vocab_k<false>(const SampleArgs&, hipStream_t);

// plain: no allowed mask, no ring, and no row with a penalty and a history.
hipError_t launch_vocab(const SampleArgs& a, bool plain, hipStream_t s) {
  return plain ? launch_vocab_k<true>(a, s) : launch_vocab_k<false>(a, s);
}

}  // namespace llmhip
