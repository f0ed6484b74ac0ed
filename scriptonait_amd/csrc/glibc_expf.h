// Bit-exact single-precision exp, restated from its published method.
//
// The reference sampler computes `(work[i] - max).exp()` with Rust's
// `f32::exp` (crates/llm-core/src/generate.rs:373), which on
// x86_64-linux-gnu lowers to glibc's `expf`. glibc (2.27 and later) uses the
// ARM optimized-routines algorithm by Szabolcs Nagy (2017, MIT/Apache-2.0):
//
//   x * N/ln2 = k + r,  N = 32, k integer (round-to-nearest via the 1.5*2^52
//   shift trick), |r| <= 1/2
//   exp(x) = 2^(k/N) * 2^(r/N)
//          ~ s * (C0 r^3 + C1 r^2 + C2 r + 1),  s = 2^(k/N) from a 32-entry
//   table of 2^(i/32) whose exponent field is patched with k/N.
//
// All internal arithmetic is in binary64 and the result is rounded once to
// binary32, so the result bits are fixed by the sequence of double
// operations. The x86_64 glibc build selects its FMA variant on CPUs with
// FMA+AVX2 and contracts `a*b + c` into one fused multiply-add, including
// both uses of `x * InvLn2N`; the fused form below reproduces that
// sequence. Tests compare this function with the host's glibc `expf` over
// every binary32 input the sampler can produce.
//
// The 32 table entries are uint64(2^(i/32)) - (i << 47), computed here from
// the mathematical definition (correctly rounded 2^(i/32)); the three
// polynomial coefficients are the published minimax coefficients of that
// algorithm, pre-divided by N^3, N^2 and N.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define LLMHIP_HD __host__ __device__ __forceinline__
#else
#define LLMHIP_HD static inline
#endif

#ifndef LLMHIP_EXPF_FUSED
#define LLMHIP_EXPF_FUSED 1
#endif

namespace llmhip {

// A constexpr table: device code reads it only with compile-time indices
// (the values become instruction immediates) and copies it to LDS.
constexpr uint64_t kExp2fTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

LLMHIP_HD uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
LLMHIP_HD float f32_from_bits(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}
LLMHIP_HD double f64_from_bits(uint64_t u) {
  double x;
  memcpy(&x, &u, 8);
  return x;
}
LLMHIP_HD uint64_t f64_bits(double x) {
  uint64_t u;
  memcpy(&u, &x, 8);
  return u;
}

// exp of a binary32 value, bit-identical to glibc 2.35's expf (FMA variant),
// with the 2^(i/32) table read from `tab` (kExp2fTab, or a copy of it that a
// kernel staged in LDS so the lookup never waits behind streaming loads).
LLMHIP_HD float glibc_expf_tab(float x, const uint64_t* tab) {
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double kShift = 0x1.8p+52;
  const double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  const double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;

  const uint32_t ux = f32_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= (f32_bits(88.0f) >> 20)) {
    // |x| >= 88, inf or nan.
    if (ux == 0xff800000u) return 0.0f;               // exp(-inf) = 0
    if (abstop >= (0x7f800000u >> 20)) return x + x;  // nan or +inf
    if (x > 0x1.62e42ep6f) return f32_from_bits(0x7f800000u);  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;                         // underflow
  }
  const double xd = (double)x;
#if LLMHIP_EXPF_FUSED
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = f64_bits(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  uint64_t t = tab[ki % 32];
  t += ki << 47;
  const double s = f64_from_bits(t);
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
#else
  double z = kInvLn2N * xd;
  double kd = z + kShift;
  const uint64_t ki = f64_bits(kd);
  kd -= kShift;
  const double r = z - kd;
  uint64_t t = tab[ki % 32];
  t += ki << 47;
  const double s = f64_from_bits(t);
  z = kC0 * r + kC1;
  const double r2 = r * r;
  double y = kC2 * r + 1.0;
  y = z * r2 + y;
  y = y * s;
  return (float)y;
#endif
}

#if !defined(__HIPCC__)
// Host form (the exhaustive comparison with glibc compiles this one).
static inline float glibc_expf(float x) { return glibc_expf_tab(x, kExp2fTab); }
#endif

}  // namespace llmhip
