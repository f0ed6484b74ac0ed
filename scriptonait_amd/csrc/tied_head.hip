// The tied output head on gfx950: logits[b][o] = dot(hidden[b], embed[o])
// for B rows and V outputs, in the reference's order, so the sampler that
// follows sees the reference's logits bit for bit.
//
// crates/llm-core/src/model.rs:396-397 computes a decode step's logits as
// ops::linear_fwd(&final_normed, &weights.embed, 1, h, vocab), whose dot
// product (crates/llm-core/src/ops/linear.rs:19-32) keeps four
// accumulators over the chunks of 4 (acc[k] += a[4j+k] * b[4j+k], a
// binary32 multiply then a binary32 add, in increasing j), folds the
// remainder's products from zero, and returns ((acc0 + acc1) + (acc2 +
// acc3)) + tail. Matching those bits rules out fused multiply-adds and
// MFMA (both round once per product-and-add), so the head runs on the
// vector ALUs at two instructions per multiply-add and is bound by them,
// not by HBM: 2*B*V*h VALU lane operations against 4*V*h bytes of embed.
//
// Tiling. A 256-thread workgroup computes 32 rows x 128 outputs. Thread
// (tr, to) = (t >> 5, t & 31) owns rows tr + 8i and outputs to + 32i
// (i < 4): 16 outputs x 4 accumulators in registers. The shared dimension
// is staged through LDS 16 floats at a time, stored k-major (float4 kq of
// row r at [kq][r]), so a wave's embed reads are 32 consecutive float4s and
// its hidden-row reads are broadcasts. Each staged chunk is read from HBM
// (or L2) once per workgroup: embed is read B/32 times in all, hidden V/128
// times.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace llmhip {

constexpr int kHeadRows = 32;     // rows per workgroup
constexpr int kHeadOuts = 128;    // outputs per workgroup
constexpr int kHeadK = 16;        // floats of the shared dimension per stage
constexpr int kHeadThreads = 256;

struct HeadArgs {
  const float* hidden;  // [B][ldh]
  const float* embed;   // [V][lde]
  float* logits;        // [B][ldl]
  uint64_t ldh, lde, ldl;
  uint32_t B, V, h;
  uint32_t row0;  // first row of this launch's grid.y tiles
};

__global__ __launch_bounds__(kHeadThreads) void tied_head_kernel(HeadArgs a) {
  __shared__ float4 xs[kHeadK / 4][kHeadRows];
  __shared__ float4 ws[kHeadK / 4][kHeadOuts];
  const uint32_t t = threadIdx.x, tr = t >> 5, to = t & 31u;
  const uint32_t o0 = blockIdx.x * kHeadOuts, r0 = a.row0 + blockIdx.y * kHeadRows;
  const uint32_t h4 = a.h & ~3u;  // the four accumulators' part; the rest is the tail

  float acc[4][4][4];  // [row i][output i][accumulator k]
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[r][o][k] = 0.0f;

  // Staging: thread t < 128 loads float4 (t & 3) of hidden row t >> 2 of
  // the tile; every thread loads float4 (t & 3) of embed rows t >> 2 and
  // 64 + (t >> 2). Floats at or past h4, and rows past B or V, read as 0:
  // a product 0 * 0 added to an accumulator leaves its value unchanged
  // (at most the sign of a zero accumulator, which no later step can see
  // in a nonzero result).
  auto load4 = [](const float* p, uint32_t k, uint32_t h4, bool row_ok) __attribute__((always_inline)) {
    if (row_ok && k + 4u <= h4) return *reinterpret_cast<const float4*>(p + k);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row_ok) {
      if (k < h4) v.x = p[k];
      if (k + 1u < h4) v.y = p[k + 1u];
      if (k + 2u < h4) v.z = p[k + 2u];
    }
    return v;
  };
  const uint32_t sq = t & 3u, sr = t >> 2;
  const float* xrow = a.hidden + (size_t)(r0 + sr) * a.ldh;
  const bool xok = t < 128u && r0 + sr < a.B;
  const float* wrow0 = a.embed + (size_t)(o0 + sr) * a.lde;
  const float* wrow1 = a.embed + (size_t)(o0 + 64u + sr) * a.lde;
  const bool wok0 = o0 + sr < a.V, wok1 = o0 + 64u + sr < a.V;
  // Vector loads need 16-byte aligned rows; otherwise dwords.
  const bool vec = ((reinterpret_cast<uintptr_t>(a.hidden) | reinterpret_cast<uintptr_t>(a.embed)) & 15u) == 0u &&
                   (a.ldh & 3u) == 0u && (a.lde & 3u) == 0u;

  for (uint32_t k0 = 0; k0 < h4; k0 += kHeadK) {
    const uint32_t k = k0 + 4u * sq;
    float4 xv, wv0, wv1;
    if (vec) {
      xv = load4(xrow, k, h4, xok);
      wv0 = load4(wrow0, k, h4, wok0);
      wv1 = load4(wrow1, k, h4, wok1);
    } else {
      auto ld1 = [&](const float* p, bool ok) __attribute__((always_inline)) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok) {
          if (k < h4) v.x = p[k];
          if (k + 1u < h4) v.y = p[k + 1u];
          if (k + 2u < h4) v.z = p[k + 2u];
          if (k + 3u < h4) v.w = p[k + 3u];
        }
        return v;
      };
      xv = ld1(xrow, xok);
      wv0 = ld1(wrow0, wok0);
      wv1 = ld1(wrow1, wok1);
    }
    __syncthreads();  // the previous stage's reads are done
    if (t < 128u) xs[sq][sr] = xv;
    ws[sq][sr] = wv0;
    ws[sq][64u + sr] = wv1;
    __syncthreads();
#pragma unroll
    for (int kq = 0; kq < kHeadK / 4; ++kq) {
      float4 xr[4], wr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xr[i] = xs[kq][tr + 8u * i];
        wr[i] = ws[kq][to + 32u * i];
      }
      // acc[k] += a[4j+k] * b[4j+k]: one product, then one add (no fused
      // multiply-add: the build keeps -ffp-contract=off).
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int o = 0; o < 4; ++o) {
          acc[r][o][0] = acc[r][o][0] + xr[r].x * wr[o].x;
          acc[r][o][1] = acc[r][o][1] + xr[r].y * wr[o].y;
          acc[r][o][2] = acc[r][o][2] + xr[r].z * wr[o].z;
          acc[r][o][3] = acc[r][o][3] + xr[r].w * wr[o].w;
        }
      }
    }
  }

  // ((acc0 + acc1) + (acc2 + acc3)) + tail; the tail (h % 4 products) is a
  // left fold from zero, read straight from the rows.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t row = r0 + tr + 8u * r;
    if (row >= a.B) continue;
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      const uint32_t out = o0 + to + 32u * o;
      if (out >= a.V) continue;
      float tail = 0.0f;
      for (uint32_t j = h4; j < a.h; ++j)
        tail = tail + a.hidden[(size_t)row * a.ldh + j] * a.embed[(size_t)out * a.lde + j];
      a.logits[(size_t)row * a.ldl + out] = ((acc[r][o][0] + acc[r][o][1]) + (acc[r][o][2] + acc[r][o][3])) + tail;
    }
  }
}

hipError_t launch_tied_head(const float* hidden, uint64_t ldh, const float* embed, uint64_t lde, float* logits,
                            uint64_t ldl, uint32_t B, uint32_t V, uint32_t h, hipStream_t s) {
  HeadArgs a{hidden, embed, logits, ldh, lde, ldl, B, V, h, 0u};
  // Row tiles go in grid.y, whose extent the device caps at 65535: a larger
  // B takes several launches, each over the next rows.
  constexpr uint32_t kMaxTilesY = 65535u;
  const uint32_t tiles = (B + kHeadRows - 1) / kHeadRows;
  for (uint32_t t0 = 0; t0 < tiles; t0 += kMaxTilesY) {
    a.row0 = t0 * kHeadRows;
    dim3 grid((V + kHeadOuts - 1) / kHeadOuts, std::min(kMaxTilesY, tiles - t0));
    hipLaunchKernelGGL(tied_head_kernel, grid, dim3(kHeadThreads), 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace llmhip
