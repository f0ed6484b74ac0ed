// gfx950 kernels of the decode-time sampler.
//
// One 1024-thread workgroup (16 wave64s) samples one row, so a batch of B
// rows is B workgroups and B=256 fills the 256 CUs of an MI355X once (the
// streaming kernel's workgroups take several rows each). Four kernels share
// the row semantics of crates/llm-core/src/generate.rs:325-420:
//
//  * sample_fast_kernel (V <= 32768, 0 < top_k <= 4096, and greedy rows):
//    the row stays in registers and the sample is decided while it streams
//    in (fast_row.h; its instantiations are compiled in fast_nch8.hip,
//    fast_nch_small.hip, fast_counts8.hip and fast_counts_small.hip).
//
//  * sample_vocab_kernel (top_k == 0 or top_k >= V: the whole vocabulary
//    is kept): the reference's three folds replayed exactly over value
//    buckets, without sorting the row (vocab_row.h; compiled in
//    vocab_full.hip and vocab_plain.hip).
//
//  * sample_stream_kernel (top-k rows past the fast kernel's V): the row
//    streamed through registers once (stream_row.h; compiled in
//    stream_topk.hip and stream_topk_bigk.hip).
//
//  * sample_general_kernel (top-k rows neither the fast nor the streaming
//    kernel takes, top_k > 4096, and rows the others hand over): an LDS select
//    of the top K, or a stable LSD radix sort of (key, id) pairs in per-row
//    HBM scratch, then the same sequential tail (general_row.h).
#include <algorithm>

#include "draw_tail.h"
#include "fast_kernel.h"
#include "fast_row.h"
#include "general_row.h"
#include "sampler_common.h"
#include "wave_ops.h"

namespace llmhip {

__global__ __launch_bounds__(kBlock) void sample_general_kernel(SampleArgs a) {
  __shared__ GenLds L;
  const uint32_t b = launch_row(a);
  if (b >= a.B) return;
  if (!a.row_cls_on && !(route_class(load_params(a, b), a.V) & a.row_class_mask)) return;
  general_row(a, b, L, false);
}

// ---------------------------------------------------------------------------
// Allowed mask in the fast kernel's slot layout: word t, bit 4c+j is set when
// the position of thread t's chunk c, float j is masked out
// (generate.rs:333-341). One workgroup; built once per call, shared by all
// rows.
// ---------------------------------------------------------------------------
template <int NCH>
__global__ __launch_bounds__(kBlock) void slotmask_kernel(SampleArgs a, uint32_t* out) {
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  uint32_t m = 0u;
  for (int c = 0; c < NCH; ++c) {
    const uint32_t base = chunk_pos<NCH>((uint32_t)c, wave, lane);
    for (int j = 0; j < 4; ++j) {
      const uint32_t p = base + j;
      if (p < a.V && masked_out(a, p)) m |= 1u << (4 * c + j);
    }
  }
  out[tid] = m;
}

// ---------------------------------------------------------------------------
// Allowed mask as bits from a corpus's tokens (Corpus::seen_tokens,
// crates/llm-core/src/corpus.rs:236-247): bit id is set when some token
// equals id < V; larger ids are ignored, as seen.get_mut(id) ignores them.
// Each workgroup ORs its share of the tokens into an LDS copy of the mask
// (repeated ids then cost LDS atomics, not global ones) and merges the
// nonzero words into the output, which a fill kernel has cleared. Masks
// larger than the LDS copy are set with global atomics directly.
// ---------------------------------------------------------------------------
constexpr uint32_t kSeenLdsWords = 16384;  // 64 KiB: masks of V <= 2^19 ids go through LDS
constexpr uint32_t kSeenMaxBlocks = 512;

__global__ __launch_bounds__(kBlock) void fill_u32_kernel(uint32_t* p, uint32_t n, uint32_t v) {
  for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) p[i] = v;
}

__global__ __launch_bounds__(kBlock) void seen_bits_kernel(const uint32_t* tokens, uint64_t n, uint32_t V,
                                                           uint32_t* bits) {
  __shared__ uint32_t m[kSeenLdsWords];
  const uint32_t words = (V + 31u) / 32u;
  const bool lds = words <= kSeenLdsWords;
  if (lds) {
    for (uint32_t i = threadIdx.x; i < words; i += kBlock) m[i] = 0u;
    __syncthreads();
  }
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const uint32_t id = tokens[i];
    if (id < V) {
      if (lds) atomicOr(&m[id >> 5], 1u << (id & 31u));
      else atomicOr(&bits[id >> 5], 1u << (id & 31u));
    }
  }
  if (lds) {
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < words; i += kBlock)
      if (m[i]) atomicOr(&bits[i], m[i]);
  }
}

// ---------------------------------------------------------------------------
// Host-side launch.
// ---------------------------------------------------------------------------
hipError_t launch_slotmask(const SampleArgs& a, uint32_t* out, hipStream_t s) {
  switch (fast_nch(a.V)) {
    case 1: hipLaunchKernelGGL(slotmask_kernel<1>, dim3(1), dim3(kBlock), 0, s, a, out); break;
    case 2: hipLaunchKernelGGL(slotmask_kernel<2>, dim3(1), dim3(kBlock), 0, s, a, out); break;
    case 4: hipLaunchKernelGGL(slotmask_kernel<4>, dim3(1), dim3(kBlock), 0, s, a, out); break;
    default: hipLaunchKernelGGL(slotmask_kernel<8>, dim3(1), dim3(kBlock), 0, s, a, out); break;
  }
  return hipGetLastError();
}

// Calls without a count table (decode steps with one: fast_counts.hip).
hipError_t launch_fast(const SampleArgs& a, bool vec, bool bigk, hipStream_t s) {
  return launch_fast_mode<false>(a, vec, bigk, s);
}

hipError_t launch_seen_bits(const uint32_t* tokens, uint64_t n, uint32_t V, uint32_t* bits, hipStream_t s) {
  const uint32_t words = (V + 31u) / 32u;
  const uint32_t fb = (uint32_t)std::min<uint64_t>((words + kBlock - 1u) / kBlock, 1024u);
  hipLaunchKernelGGL(fill_u32_kernel, dim3(fb), dim3(kBlock), 0, s, bits, words, 0u);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || n == 0) return e;
  const uint64_t per = words <= kSeenLdsWords ? 16u * kBlock : (uint64_t)kBlock;  // tokens per block and pass
  const uint32_t blocks = (uint32_t)std::min<uint64_t>((n + per - 1u) / per, kSeenMaxBlocks);
  hipLaunchKernelGGL(seen_bits_kernel, dim3(blocks), dim3(kBlock), 0, s, tokens, n, V, bits);
  return hipGetLastError();
}

// Moves the device-entry flags and the hand-over count to words[kStatusTakenWord ..
// +1] and clears them, each in one atomic exchange: a kernel on another stream
// that sets a flag or counts a hand-over meanwhile is either taken now or
// left for the next call, never lost.
__global__ void take_status_kernel(uint32_t* words) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    words[kStatusTakenWord] = atomicExch(&words[kStatusDeviceWord], 0u);
    words[kStatusTakenWord + 1] = atomicExch(&words[kStatusHandoverWord], 0u);
  }
}

hipError_t launch_take_status(uint32_t* words, hipStream_t s) {
  hipLaunchKernelGGL(take_status_kernel, dim3(1), dim3(64), 0, s, words);
  return hipGetLastError();
}

hipError_t launch_general(const SampleArgs& a, hipStream_t s) {
  const uint32_t grid = launch_grid(a);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(sample_general_kernel, dim3(grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace llmhip
