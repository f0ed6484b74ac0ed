// Wavefront (64-lane) building blocks for gfx950.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmhip {

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

// DPP move: lanes whose source is outside the pattern (or rows outside
// ROW_MASK) read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp0(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xf, false);
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP: row_shr 1,2,4,8
// within each row of 16, then row_bcast:15 and row_bcast:31 across rows.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += dpp0<0x111>(x);
  x += dpp0<0x112>(x);
  x += dpp0<0x114>(x);
  x += dpp0<0x118>(x);
  x += dpp0<0x142, 0xa>(x);
  x += dpp0<0x143, 0xc>(x);
  return x;
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp0_f64(double x) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = dpp0<CTRL, ROW_MASK>((uint32_t)u), hi = dpp0<CTRL, ROW_MASK>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// The same prefix sum in f64 (lanes read +0.0 where the pattern has no
// source).
__device__ __forceinline__ double wave_incl_scan_f64(double x) {
  x += dpp0_f64<0x111>(x);
  x += dpp0_f64<0x112>(x);
  x += dpp0_f64<0x114>(x);
  x += dpp0_f64<0x118>(x);
  x += dpp0_f64<0x142, 0xa>(x);
  x += dpp0_f64<0x143, 0xc>(x);
  return x;
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t x) {
#pragma unroll
  for (uint32_t off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
#pragma unroll
  for (uint32_t off = 32; off > 0; off >>= 1) {
    const uint32_t y = __shfl_xor(x, off, 64);
    x = y > x ? y : x;
  }
  return x;
}

// Value of `x` held by lane `l` (l uniform across the wave).
__device__ __forceinline__ float readlane_f32(float x, uint32_t l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), (int)l));
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t x, uint32_t l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)x, (int)l);
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t x, uint32_t l) {
  const uint32_t lo = readlane_u32((uint32_t)x, l), hi = readlane_u32((uint32_t)(x >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ double readlane_f64(double x, uint32_t l) {
  return __longlong_as_double((long long)readlane_u64((uint64_t)__double_as_longlong(x), l));
}

// Number of set bits of the wave mask m in lanes below this one.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return (uint32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Bit mask of the lanes below this one.
__device__ __forceinline__ uint64_t lanemask_lt() {
  const uint32_t lane = lane_id();
  return lane == 0 ? 0ull : (~0ull >> (64u - lane));
}

// atomicAdd(&bins[bin], 1) for every active lane of the wave. The lanes that
// share the first active lane's bin add as one atomic, so lanes whose bins
// crowd one address do not serialize there.
__device__ __forceinline__ void bin_add_grouped(uint32_t* bins, uint32_t bin) {
  const uint64_t act = __ballot(true);
  const uint32_t lead = (uint32_t)__ffsll((unsigned long long)act) - 1u;
  const uint32_t b0 = readlane_u32(bin, lead);
  const uint64_t m = __ballot(bin == b0);
  if (bin != b0) atomicAdd(&bins[bin], 1u);
  else if (lane_id() == lead) atomicAdd(&bins[b0], (uint32_t)__popcll(m));
}

// "Better" for the greedy argmax (crates/llm-core/src/ops/loss.rs:6-16):
// larger value wins; equal values keep the smaller index.
__device__ __forceinline__ void argmax_combine(float& bv, uint32_t& bi, float ov, uint32_t oi) {
  if (ov > bv || (ov == bv && oi < bi)) {
    bv = ov;
    bi = oi;
  }
}

__device__ __forceinline__ void wave_argmax(float& bv, uint32_t& bi) {
#pragma unroll
  for (uint32_t off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const uint32_t oi = __shfl_xor(bi, off, 64);
    argmax_combine(bv, bi, ov, oi);
  }
}

}  // namespace llmhip
