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

// key_at(i) / id_at(i): i-th candidate (i < n) in sorted order; st is row
// b's RNG state and tab the exp table (kExp2fTab or an LDS copy of it).
// Must be called by all 64 lanes of exactly one wave. Writes out_ids,
// rng_state, out_kept and (if requested) out_probs for row b.
template <class KeyAt, class IdAt>
__device__ __forceinline__ void draw_tail(const SampleArgs& a, uint32_t b, const llmhip_params& P, uint32_t n,
                          KeyAt key_at, IdAt id_at, uint64_t st, const uint64_t* tab) {
  const uint32_t lane = lane_id();
  const uint32_t k0 = key_at(0);
  // fold(NEG_INFINITY, f32::max) over sorted candidates: the first one
  // unless it is NaN (NaN keys sort last, so then all are NaN).
  const float mx = k0 <= kKeyNaN ? -INFINITY : key2f(k0);
  auto e_at = [&](uint32_t i) { return glibc_expf_tab(key2f(key_at(i)) - mx, tab); };

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

// Same computation for n <= 64 candidates held one per lane (lane i holds
// candidate i's key and id; lanes >= n are ignored), with the RNG state
// already in a register. Each fold is a chain of dependent VGPR adds over
// all 64 values, fetched from LDS (`buf`, 128 floats) into registers up
// front; padding lanes contribute +0.0, which leaves an f32 sum of
// non-negative terms unchanged. Running values are parked in LDS so that
// lane i can test its own prefix, and a ballot finds the first lane that
// decides (the reference's early `break`).
__device__ __forceinline__ void draw_tail_small(const SampleArgs& a, uint32_t b, const llmhip_params& P,
                                                uint32_t n, uint32_t my_key, uint32_t my_id,
                                                uint64_t st, float* buf, const uint64_t* tab) {
  const uint32_t lane = lane_id();
  const bool act = lane < n;
  const uint32_t k0 = readlane_u32(my_key, 0);
  const float mx = k0 <= kKeyNaN ? -INFINITY : key2f(k0);
  const float e = act ? glibc_expf_tab(key2f(my_key) - mx, tab) : 0.0f;
  float* cbuf = buf + 64;
  const float4* b4 = reinterpret_cast<const float4*>(buf);

  // generate.rs:374
  buf[lane] = e;
  float sum = 0.0f;
  {
    float4 v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = b4[q];
    bool go = true;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (go) {
        sum += v[q].x;
        sum += v[q].y;
        sum += v[q].z;
        sum += v[q].w;
        if ((q & 1) && 4u * (q + 1) >= n) go = false;
      }
    }
  }
  // generate.rs:375-377
  if (!(sum > 0.0f) || !isfinite(sum)) {
    if (lane == 0) {
      a.out_ids[b] = n > 0 ? my_id : 0u;
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }
  const float p = act ? e / sum : 0.0f;  // generate.rs:378-380

  // generate.rs:384-395
  uint32_t keep = n;
  if (P.min_p > 0.0f) {
    const float thr = P.min_p * readlane_f32(p, 0);
    const uint64_t fail = __ballot(act && !(p >= thr));
    if (fail) keep = (uint32_t)__ffsll((unsigned long long)fail) - 1u;
    if (keep < 1u) keep = 1u;
  }

  // generate.rs:397-411: c_i = fold of p_0..p_i; lane i reads its c_i. The
  // total over a kept prefix is that fold at its last element.
  buf[lane] = p;
  float4 pv[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) pv[q] = b4[q];
  {
    // Stops after the block of 8 where the fold reaches top_p (every lane
    // holds the same running value, so the exit is uniform).
    const float tp = P.top_p < 1.0f ? P.top_p : INFINITY;
    float c = 0.0f;
    bool go = true;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (go) {
        float4 o;
        c += pv[q].x;
        o.x = c;
        c += pv[q].y;
        o.y = c;
        c += pv[q].z;
        o.z = c;
        c += pv[q].w;
        o.w = c;
        if (lane == 0) reinterpret_cast<float4*>(cbuf)[q] = o;
        // c is the same in every lane: read it as a scalar.
        if ((q & 1) && (4u * (q + 1) >= keep || __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(c))) >= tp)) go = false;
      }
    }
  }
  const float my_c = lane < keep ? cbuf[lane] : 0.0f;
  uint32_t stop = keep;
  if (P.top_p < 1.0f) {
    const uint64_t hit = __ballot(lane < keep && my_c >= P.top_p);
    if (hit) stop = (uint32_t)__ffsll((unsigned long long)hit);
  }
  const float total = readlane_f32(my_c, stop - 1u);

  // generate.rs:412-419: r_i = r before subtracting p_i; lane i tests r_i < p_i.
  const float ur = next_f32(st);
  {
    // r - p < 0 exactly when r < p, so r turns negative at the pick: stop
    // after that block of 8.
    float r = ur * total;
    bool go = true;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (go) {
        float4 o;
        o.x = r;
        r -= pv[q].x;
        o.y = r;
        r -= pv[q].y;
        o.z = r;
        r -= pv[q].z;
        o.w = r;
        r -= pv[q].w;
        if (lane == 0) reinterpret_cast<float4*>(cbuf)[q] = o;
        if ((q & 1) && (4u * (q + 1) >= stop || __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(r))) < 0.0f)) go = false;
      }
    }
  }
  const float my_r = lane < stop ? cbuf[lane] : 0.0f;
  const uint64_t hit = __ballot(lane < stop && my_r < p);
  const uint32_t pick = hit ? (uint32_t)__ffsll((unsigned long long)hit) - 1u : stop - 1u;
  const uint32_t id = readlane_u32(my_id, pick);
  if (lane == 0) {
    a.out_ids[b] = id;
    a.rng_state[b] = st;
    if (a.out_kept) a.out_kept[b] = stop;
  }
  if (a.out_probs && lane < stop) a.out_probs[(size_t)b * a.V + my_id] = p;
}

}  // namespace llmhip
