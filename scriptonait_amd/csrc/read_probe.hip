// The achievable streaming-read floor for the fast kernel's access shape: a
// measurement kernel, not part of the sampler. Built into libllmhip_probe.so
// and run by bench.py --read-floor.
//
// read_floor_kernel reads B rows of V floats exactly as sample_fast_kernel<8>
// does (one 1024-thread workgroup per row; lane l of wave w loads floats
// 4l..4l+3 of the 1 KiB block c*16 + w for chunks c = 0..7, one nontemporal
// dwordx4 each; positions past V read position 0) and keeps the loads alive
// with a comparison that never holds.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

constexpr int kProbeChunks = 8;
constexpr uint32_t kProbeBlock = 1024;

__global__ __launch_bounds__(kProbeBlock) void read_floor_kernel(const float* x, uint64_t ld, uint32_t V, float* out) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const float* row = x + (size_t)blockIdx.x * ld;
  f4v v[kProbeChunks];
#pragma unroll
  for (int c = 0; c < kProbeChunks; ++c) {
    const uint32_t base = ((uint32_t)c * 16u + wave) * 256u + lane * 4u;
    v[c] = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(row + (base + 3u < V ? base : 0u)));
  }
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < kProbeChunks; ++c) m = fmaxf(m, fmaxf(fmaxf(v[c].x, v[c].y), fmaxf(v[c].z, v[c].w)));
  if (m == 1234567.0f) out[blockIdx.x] = m;  // never taken for the probe's inputs
}

}  // namespace

extern "C" {

// Launch read_floor_kernel over B rows (V <= 32768, ld % 4 == 0, 16-byte
// aligned rows). Returns a hipError_t value.
int llmhip_probe_read(const float* x, size_t B, size_t V, size_t ld, float* out, void* stream) {
  if (!x || !out || B == 0 || V == 0 || V > (size_t)kProbeChunks * 16u * 256u || ld < V || ld % 4u != 0u ||
      (reinterpret_cast<uintptr_t>(x) % 16u) != 0u)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(read_floor_kernel, dim3((uint32_t)B), dim3(kProbeBlock), 0, static_cast<hipStream_t>(stream), x,
                     (uint64_t)ld, (uint32_t)V, out);
  return (int)hipGetLastError();
}

}  // extern "C"
