// The sequential end of sample_with, run by one wavefront over a candidate
// list already sorted by (value desc, id asc).
//
// crates/llm-core/src/generate.rs:372-419: max, expf, the softmax sum as a
// left fold in sorted order, normalization, min-p prefix, top-p cumulative
// fold, and the inverse-CDF walk driven by one SplitMix64 step. Every f32
// operation is the reference's, in the reference's order: the folds are
// replayed one element at a time (v_readlane broadcasts element t to the
// whole wave, which adds it), so the rounding sequence is identical.
#pragma once
#include "sampler_common.h"
#include "wave_ops.h"

namespace llmhip {

// key_at(i) / id_at(i): i-th candidate (i < n) in sorted order.
// Must be called by all 64 lanes of exactly one wave. Writes out_ids,
// rng_state, out_kept and (if requested) out_probs for row b.
template <class KeyAt, class IdAt>
__device__ void draw_tail(const SampleArgs& a, uint32_t b, const llmhip_params& P, uint32_t n,
                          KeyAt key_at, IdAt id_at) {
  const uint32_t lane = lane_id();
  const uint32_t k0 = key_at(0);
  // fold(NEG_INFINITY, f32::max) over sorted candidates: the first one
  // unless it is NaN (NaN keys sort last, so then all are NaN).
  const float mx = k0 <= kKeyNaN ? -INFINITY : key2f(k0);
  auto e_at = [&](uint32_t i) { return glibc_expf(key2f(key_at(i)) - mx); };

  // generate.rs:374: sum as a left fold in sorted order.
  float sum = 0.0f;
  for (uint32_t c = 0; c < n; c += 64) {
    const uint32_t i = c + lane;
    const float e = i < n ? e_at(i) : 0.0f;
    const uint32_t m = min(64u, n - c);
    for (uint32_t t = 0; t < m; ++t) sum += readlane_f32(e, t);
  }
  // generate.rs:375-377: degenerate exit, no draw.
  if (!(sum > 0.0f) || !isfinite(sum)) {
    if (lane == 0) {
      a.out_ids[b] = n > 0 ? id_at(0) : 0u;
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }
  auto p_at = [&](uint32_t i) { return e_at(i) / sum; };  // generate.rs:378-380

  uint32_t keep = n;
  // generate.rs:384-395: longest prefix with p >= min_p * p_0, at least 1.
  if (P.min_p > 0.0f) {
    const float thr = P.min_p * p_at(0);
    for (uint32_t c = 0; c < n; c += 64) {
      const uint32_t i = c + lane;
      const bool fail = i < n && !(p_at(i) >= thr);
      const uint64_t mask = __ballot(fail);
      if (mask) {
        keep = c + (uint32_t)__ffsll((unsigned long long)mask) - 1u;
        break;
      }
    }
    if (keep < 1u) keep = 1u;
  }

  // generate.rs:397-409 (top-p) and :411 (total). When top-p is on, the
  // total over the kept prefix is the same left fold the cumulative ran.
  float total = 0.0f;
  if (P.top_p < 1.0f) {
    uint32_t kp = keep;
    bool hit = false;
    for (uint32_t c = 0; c < keep && !hit; c += 64) {
      const uint32_t i = c + lane;
      const float p = i < keep ? p_at(i) : 0.0f;
      const uint32_t m = min(64u, keep - c);
      for (uint32_t t = 0; t < m; ++t) {
        total += readlane_f32(p, t);
        if (total >= P.top_p) {
          kp = c + t + 1u;
          hit = true;
          break;
        }
      }
    }
    keep = kp;
  } else {
    for (uint32_t c = 0; c < keep; c += 64) {
      const uint32_t i = c + lane;
      const float p = i < keep ? p_at(i) : 0.0f;
      const uint32_t m = min(64u, keep - c);
      for (uint32_t t = 0; t < m; ++t) total += readlane_f32(p, t);
    }
  }

  // generate.rs:412-419: r = u * total, walk with r -= p.
  uint64_t st = a.rng_state[b];
  const float u = next_f32(st);
  float r = u * total;
  uint32_t pick = keep - 1u;
  bool found = false;
  for (uint32_t c = 0; c < keep && !found; c += 64) {
    const uint32_t i = c + lane;
    const float p = i < keep ? p_at(i) : 0.0f;
    const uint32_t m = min(64u, keep - c);
    for (uint32_t t = 0; t < m; ++t) {
      const float pv = readlane_f32(p, t);
      if (r < pv) {
        pick = c + t;
        found = true;
        break;
      }
      r -= pv;
    }
  }
  if (lane == 0) {
    a.out_ids[b] = id_at(pick);
    a.rng_state[b] = st;
    if (a.out_kept) a.out_kept[b] = keep;
  }
  if (a.out_probs) {
    float* prow = a.out_probs + (size_t)b * a.V;
    for (uint32_t i = lane; i < keep; i += 64) prow[id_at(i)] = p_at(i);
  }
}

}  // namespace llmhip
