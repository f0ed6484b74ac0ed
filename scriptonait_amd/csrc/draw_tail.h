// The sequential end of sample_with, run by one wavefront over a candidate
// list already sorted by (value desc, id asc).
//
// crates/llm-core/src/generate.rs:372-419: max, expf, the softmax sum as a
// left fold in sorted order, normalization, min-p prefix, top-p cumulative
// fold, and the inverse-CDF walk driven by one SplitMix64 step. Every f32
// operation is the reference's, in the reference's order: each fold adds
// (or subtracts) the terms one at a time, read from LDS as broadcasts, so
// the rounding sequence is identical.
//
// Common contract: key_at(i) / id_at(i) give the i-th candidate (i < n) in
// sorted order; st is row b's RNG state, tab the exp table (an LDS copy of
// kExp2fTab) and len_b the row's ring length (decode-step mode). Each tail
// must be called by all 64 lanes of exactly one wave and writes out_ids,
// rng_state, out_kept and (if requested) out_probs for row b. The max is
// the first key unless it is NaN (NaN keys sort last, so then all are NaN).
#pragma once
#include "sampler_common.h"
#include "wave_ops.h"

// Profiling hook: a profiling build defines LLMHIP_TAIL_MARK(i) (a
// timestamp at step i of the register tail); empty otherwise.
#ifndef LLMHIP_TAIL_MARK
#define LLMHIP_TAIL_MARK(i)
#endif

namespace llmhip {

// generate.rs:372-373: buf[i] = expf(w_i - max) for the n sorted
// candidates (the max is the first key, or -inf when the keys are NaN), and
// +0.0 up to n rounded to 64. Threads first, first + stride, ... share it.
template <class KeyAt>
__device__ __forceinline__ void stage_exp_terms(float* buf, uint32_t n, KeyAt key_at, const uint64_t* tab,
                                                uint32_t first, uint32_t stride) {
  const uint32_t k0 = key_at(0);
  const float mx = k0 <= kKeyNaN ? -INFINITY : key2f(k0);
  const uint32_t nr = (n + 63u) & ~63u;
  for (uint32_t i = first; i < nr; i += stride) buf[i] = i < n ? glibc_expf_tab(key2f(key_at(i)) - mx, tab) : 0.0f;
}

// The same computation for n <= 4096 candidates, with the terms staged in
// LDS (`buf`: n rounded up to 64 floats, 16-byte aligned; STAGED: the
// caller has staged them, by stage_exp_terms). Every fold is the
// reference's left fold in f32, read as broadcast float4s: the softmax sum
// 16 terms per step, top-p and the walk in blocks of 8 whose last value is
// tested (c never decreases; r - p < 0 exactly when r < p), the block that
// decides being resolved once, one lane per term. Terms past the kept
// prefix are set to +0.0, which leaves either fold unchanged.
// Must be called by all 64 lanes of exactly one wave.
template <bool STAGED = false, class KeyAt, class IdAt>
__device__ __forceinline__ void draw_tail_lds(const SampleArgs& a, uint32_t b, uint32_t len_b, const llmhip_params& P,
                                              uint32_t n, KeyAt key_at, IdAt id_at, uint64_t st, const uint64_t* tab,
                                              float* buf) {
  const uint32_t lane = lane_id();
  const uint32_t nr = (n + 63u) & ~63u;
  if (!STAGED) stage_exp_terms(buf, n, key_at, tab, lane, 64u);
  const float4* b4 = reinterpret_cast<const float4*>(buf);
  auto t8_at = [&](uint32_t base, float (&t8)[8]) __attribute__((always_inline)) {
    const float4 lo = b4[base / 4u], hi = b4[base / 4u + 1u];
    t8[0] = lo.x; t8[1] = lo.y; t8[2] = lo.z; t8[3] = lo.w;
    t8[4] = hi.x; t8[5] = hi.y; t8[6] = hi.z; t8[7] = hi.w;
  };

  // generate.rs:374: sum = ((0 + e_0) + e_1) + ... . Term by term over the
  // float4s [q0, q1) (a multiple of 4 apart), the next 16 terms loading while
  // the current 16 are added.
  float sum = 0.0f;
  auto add_terms = [&](uint32_t q0, uint32_t q1) __attribute__((always_inline)) {
    float4 c0 = b4[q0], c1 = b4[q0 + 1u], c2 = b4[q0 + 2u], c3 = b4[q0 + 3u];
    for (uint32_t q = q0; q < q1; q += 4u) {
      float4 d0 = c0, d1 = c1, d2 = c2, d3 = c3;
      if (q + 4u < q1) {
        d0 = b4[q + 4u];
        d1 = b4[q + 5u];
        d2 = b4[q + 6u];
        d3 = b4[q + 7u];
      }
      sum += c0.x; sum += c0.y; sum += c0.z; sum += c0.w;
      sum += c1.x; sum += c1.y; sum += c1.z; sum += c1.w;
      sum += c2.x; sum += c2.y; sum += c2.z; sum += c2.w;
      sum += c3.x; sum += c3.y; sum += c3.z; sum += c3.w;
      c0 = d0; c1 = d1; c2 = d2; c3 = d3;
    }
  };
  // The first 64 terms one at a time (the sum passes through its first
  // binades there). Then 64 at a time: while the sum S stays in its binade
  // [2^E, 2^(E+1)), fl(S + t) = S + rne(t / u) * u with u = 2^(E-23), an
  // integer count of ulps that does not depend on S, except at an exact
  // half-ulp tie, where round-half-even looks at S's last bit. A block with
  // no such tie whose counts keep S in its binade adds their total at once
  // (exact: S / u + total < 2^24); any other block (a binade change, a tie, a
  // term or sum that is not finite) is added term by term.
  add_terms(0u, min(nr, 64u) / 4u);
  for (uint32_t base = 64u; base < nr; base += 64u) {
    const float t = buf[base + lane];
    bool step = !(sum >= 1.0f) || !isfinite(sum);
    if (!step) {
      const int E = (int)((__float_as_uint(sum) >> 23) & 0xffu) - 127;  // sum is normal, >= 1
      const float q = ldexpf(t, 23 - E);                                 // t / u, exact
      const float r = rintf(q);
      const bool odd = !isfinite(t) || q - floorf(q) == 0.5f;
      const uint32_t tot = readlane_u32(wave_incl_scan((uint32_t)r), 63u);
      const uint32_t si = (uint32_t)ldexpf(sum, 23 - E);  // S / u, in [2^23, 2^24)
      step = __ballot(odd) != 0ull || si + tot >= (1u << 24);
      if (!step) sum = ldexpf((float)(si + tot), E - 23);
    }
    if (step) add_terms(base / 4u, base / 4u + 16u);
  }
  // generate.rs:375-377: degenerate exit, no draw.
  if (!(sum > 0.0f) || !isfinite(sum)) {
    if (lane == 0) {
      store_result(a, b, id_at(0), len_b);
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }
  // generate.rs:378-380: p_i = e_i / sum, and generate.rs:384-395: the
  // longest prefix with p >= min_p * p_0, at least 1. With min-p, p_i is
  // computed only as far as that prefix reaches: the terms past it are
  // cleared below.
  uint32_t keep = n;
  if (P.min_p > 0.0f) {
    const float thr = P.min_p * (buf[0] / sum);
    for (uint32_t c = 0; c < n; c += 64u) {
      const uint32_t i = c + lane;
      float p = 0.0f;
      if (i < n) {
        p = buf[i] / sum;
        buf[i] = p;
      }
      const uint64_t fail = __ballot(i < n && !(p >= thr));
      if (fail) {
        keep = c + (uint32_t)__ffsll((unsigned long long)fail) - 1u;
        break;
      }
    }
    if (keep < 1u) keep = 1u;
  } else {
    for (uint32_t i = lane; i < n; i += 64u) buf[i] = buf[i] / sum;
  }
  for (uint32_t i = keep + lane; i < nr; i += 64u) buf[i] = 0.0f;

  // The top-p and walk folds below run 64 terms at a time in integer ulps
  // where they can, as the softmax sum does: inside a binade and with no
  // half-ulp tie, each step adds (or subtracts) rne(p / u) ulps, so a wave
  // scan of those counts gives every running value of the block exactly.
  // A block where that does not hold runs term by term.
  auto ulp_exp = [](float x) __attribute__((always_inline)) {  // x normal: x in [2^E, 2^(E+1))
    return (int)((__float_as_uint(x) >> 23) & 0xffu) - 127;
  };

  // generate.rs:397-411: c_i = ((0 + p_0) + ...) + p_i; the cut is the first
  // c_i >= top_p (all of the prefix when top_p >= 1 or never reached); the
  // total is the fold at the last kept term.
  uint32_t stop = keep;
  float total = 0.0f;
  if (__builtin_expect(keep <= 64u, 1)) {  // one block: term by term, in a compact loop
    const float tp = P.top_p < 1.0f ? P.top_p : INFINITY;
    float c = 0.0f, cprev = 0.0f;
    uint32_t k8 = 0u;
    for (uint32_t base = 0; base < keep; base += 8u) {
      float t8[8];
      t8_at(base, t8);
      cprev = c;
#pragma unroll
      for (int j = 0; j < 8; ++j) c += t8[j];
      k8 = base;
      if (c >= tp) break;
    }
    // Lane j < 8 recomputes c_{k8+j} from the block's start, in order.
    float t8[8], t = cprev;
    t8_at(k8, t8);
#pragma unroll
    for (int j = 0; j < 8; ++j) t = (uint32_t)j <= lane ? t + t8[j] : t;
    const uint64_t hit = __ballot(lane < 8u && k8 + lane < keep && t >= tp);
    if (hit) stop = k8 + (uint32_t)__ffsll((unsigned long long)hit);
    total = readlane_f32(t, stop - 1u - k8);
  } else {
    const float tp = P.top_p < 1.0f ? P.top_p : INFINITY;
    float c = 0.0f;
    bool done = false;
    // Term by term over [b0, b0 + 64): blocks of 8 whose last value is
    // tested; the block with the cut (or with the end of the kept prefix) is
    // resolved by lanes j < 8, each recomputing c_{base+j} from its start.
    auto fold_terms = [&](uint32_t b0) __attribute__((always_inline)) {
      for (uint32_t base = b0; base < b0 + 64u; base += 8u) {
        float t8[8];
        t8_at(base, t8);
        const float cprev = c;
#pragma unroll
        for (int j = 0; j < 8; ++j) c += t8[j];
        if (c >= tp || base + 8u >= keep) {
          float t = cprev;
#pragma unroll
          for (int j = 0; j < 8; ++j) t = (uint32_t)j <= lane ? t + t8[j] : t;
          const uint64_t hit = __ballot(lane < 8u && base + lane < keep && t >= tp);
          stop = hit ? base + (uint32_t)__ffsll((unsigned long long)hit) : keep;
          total = readlane_f32(t, stop - 1u - base);
          done = true;
          return;
        }
      }
    };
    const uint32_t kr = (keep + 63u) & ~63u;
    for (uint32_t b0 = 0u; b0 < kr && !done; b0 += 64u) {
      // The first block term by term (c starts at 0 and climbs through
      // binades), and a block with few kept terms left (a scan costs about
      // as much as 30 steps).
      bool step = b0 == 0u || keep - b0 < 32u || !(c >= 0x1p-126f) || !isfinite(c);
      if (!step) {
        const float pj = buf[b0 + lane];  // 0 past keep
        const int E = ulp_exp(c);
        const float q = ldexpf(pj, 23 - E);  // p / u, exact (p <= p_0 <= c)
        const float rq = rintf(q);
        const uint32_t P = wave_incl_scan((uint32_t)rq);
        const uint32_t ci = (uint32_t)ldexpf(c, 23 - E);  // c / u, in [2^23, 2^24)
        step = __ballot(q - floorf(q) == 0.5f) != 0ull || ci + readlane_u32(P, 63u) >= (1u << 24);
        if (!step) {
          const float cj = ldexpf((float)(ci + P), E - 23);  // c after term b0 + lane
          const uint64_t hit = __ballot(b0 + lane < keep && cj >= tp);
          if (hit) {
            const uint32_t j = (uint32_t)__ffsll((unsigned long long)hit) - 1u;
            stop = b0 + j + 1u;
            total = readlane_f32(cj, j);
            done = true;
          } else {
            c = readlane_f32(cj, 63u);
          }
        }
      }
      if (step) fold_terms(b0);
    }
    if (!done) total = c;  // the kept prefix ended in a block added in ulps
  }
  // Terms past the cut leave the walk's r unchanged too.
  for (uint32_t i = stop + lane; i < keep; i += 64u) buf[i] = 0.0f;

  // generate.rs:412-419: r_0 = u * total; step i tests r_i < p_i, then
  // subtracts p_i; no hit picks the last kept term.
  const float u = next_f32(st);
  uint32_t pick = stop - 1u;
  if (__builtin_expect(stop <= 64u, 1)) {  // one block: term by term, in a compact loop
    float r = u * total, rprev = r;
    uint32_t k8 = 0u;
    bool neg = false;
    for (uint32_t base = 0; base < stop; base += 8u) {
      float t8[8];
      t8_at(base, t8);
      rprev = r;
#pragma unroll
      for (int j = 0; j < 8; ++j) r -= t8[j];
      k8 = base;
      if (r < 0.0f) {
        neg = true;
        break;
      }
    }
    if (neg) {
      // Lane j < 8 recomputes r_{k8+j} (before its own subtraction).
      float t8[8], t = rprev;
      t8_at(k8, t8);
#pragma unroll
      for (int j = 0; j < 8; ++j) t = (uint32_t)j < lane ? t - t8[j] : t;
      const float pj = lane < 8u ? buf[k8 + lane] : 0.0f;
      const uint64_t hit = __ballot(lane < 8u && k8 + lane < stop && t < pj);
      if (hit) pick = k8 + (uint32_t)__ffsll((unsigned long long)hit) - 1u;
    }
  } else {
    float r = u * total;
    bool found = false;
    // Term by term over [b0, b0 + 64): blocks of 8 whose last value is tested
    // (r_i - p_i < 0 exactly when r_i < p_i), the deciding block resolved by
    // lanes j < 8, each recomputing r_{base+j} before its own subtraction.
    auto walk_terms = [&](uint32_t b0) __attribute__((always_inline)) {
      for (uint32_t base = b0; base < b0 + 64u && base < stop; base += 8u) {
        float t8[8];
        t8_at(base, t8);
        const float rprev = r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r -= t8[j];
        if (r < 0.0f) {
          float t = rprev;
#pragma unroll
          for (int j = 0; j < 8; ++j) t = (uint32_t)j < lane ? t - t8[j] : t;
          const float pj = lane < 8u ? buf[base + lane] : 0.0f;
          const uint64_t hit = __ballot(lane < 8u && base + lane < stop && t < pj);
          if (hit) pick = base + (uint32_t)__ffsll((unsigned long long)hit) - 1u;
          found = true;
          return;
        }
      }
    };
    const uint32_t sr = (stop + 63u) & ~63u;
    for (uint32_t b0 = 0u; b0 < sr && !found; b0 += 64u) {
      // Term by term: the first block of a short walk (it usually ends
      // there), and a block with few terms left.
      bool step = (b0 == 0u && stop <= 256u) || stop - b0 < 32u || !(r >= 0x1p-126f) || !isfinite(r);
      if (!step) {
        const float pj = buf[b0 + lane];  // 0 past stop
        const int E = ulp_exp(r);
        const float q = ldexpf(pj, 23 - E);
        // p can exceed r by far here (the pick): counts of 2^25 and more are
        // clamped, which keeps the scan from wrapping; every lane after such
        // a term fails the bound below, and its own test hits.
        const float rq = rintf(fminf(q, 0x1p25f));
        const uint32_t qi = (uint32_t)rq;
        const uint32_t Pi = wave_incl_scan(qi), Pe = Pi - qi;
        const uint32_t ri = (uint32_t)ldexpf(r, 23 - E);  // r / u, in [2^23, 2^24)
        const uint64_t ties = __ballot(q - floorf(q) == 0.5f);
        // r before lane j's test is exact while no tie comes before j and
        // every value so far stays a whole ulp above 2^E (below it the
        // spacing halves): the lanes where that holds are a prefix [0, v).
        const bool ok = (ties & lanemask_lt()) == 0ull && Pe < ri - (1u << 23);
        const uint64_t okm = __ballot(ok);
        const uint32_t v = okm == ~0ull ? 64u : (uint32_t)__ffsll((unsigned long long)~okm) - 1u;
        const float rb = ldexpf((float)(ri - Pe), E - 23);
        const uint64_t hit = __ballot(lane < v && b0 + lane < stop && rb < pj);
        const uint32_t tot = readlane_u32(Pi, 63u);
        if (hit) {
          pick = b0 + (uint32_t)__ffsll((unsigned long long)hit) - 1u;
          found = true;
        } else if (v == 64u && ties == 0ull && tot < ri - (1u << 23)) {
          r = ldexpf((float)(ri - tot), E - 23);
        } else {
          step = true;
        }
      }
      if (step) walk_terms(b0);
    }
  }
  if (lane == 0) {
    store_result(a, b, id_at(pick), len_b);
    a.rng_state[b] = st;
    if (a.out_kept) a.out_kept[b] = stop;
  }
  if (a.out_probs) {
    float* prow = a.out_probs + (size_t)b * a.V;
    for (uint32_t i = lane; i < stop; i += 64u) prow[id_at(i)] = buf[i];
  }
}

// The same computation for any n, with the terms staged in LDS windows of
// `cap` floats (a multiple of 64; `buf` 16-byte aligned): each fold runs
// over the windows in order with its value carried from one to the next,
// and a window's terms are recomputed from the keys when it is staged.
// Used where n exceeds what one window holds.
template <class KeyAt, class IdAt>
__device__ __forceinline__ void draw_tail_win(const SampleArgs& a, uint32_t b, uint32_t len_b, const llmhip_params& P,
                                              uint32_t n, KeyAt key_at, IdAt id_at, uint64_t st, const uint64_t* tab,
                                              float* buf, uint32_t cap) {
  const uint32_t lane = lane_id();
  const uint32_t k0 = key_at(0);
  const float mx = k0 <= kKeyNaN ? -INFINITY : key2f(k0);
  auto e_at = [&](uint32_t i) { return glibc_expf_tab(key2f(key_at(i)) - mx, tab); };
  const float4* b4 = reinterpret_cast<const float4*>(buf);
  // buf[j] = the term of i = w0 + j for i < lim (e_i, or e_i / div when div
  // is not 0), +0.0 up to the next multiple of 64. Returns the count staged.
  auto stage = [&](uint32_t w0, uint32_t lim, float div) __attribute__((always_inline)) {
    const uint32_t cnt = min(cap, lim - w0), cr = (cnt + 63u) & ~63u;
    for (uint32_t j = lane; j < cr; j += 64u) {
      float t = 0.0f;
      if (j < cnt) {
        t = e_at(w0 + j);
        if (div != 0.0f) t = t / div;
      }
      buf[j] = t;
    }
    return cnt;
  };
  auto t8_at = [&](uint32_t base, float (&t8)[8]) __attribute__((always_inline)) {
    const float4 lo = b4[base / 4u], hi = b4[base / 4u + 1u];
    t8[0] = lo.x; t8[1] = lo.y; t8[2] = lo.z; t8[3] = lo.w;
    t8[4] = hi.x; t8[5] = hi.y; t8[6] = hi.z; t8[7] = hi.w;
  };

  // generate.rs:374: the softmax sum as one left fold over the windows.
  float sum = 0.0f;
  for (uint32_t w0 = 0; w0 < n; w0 += cap) {
    const uint32_t cnt = stage(w0, n, 0.0f);
    for (uint32_t base = 0; base < cnt; base += 8u) {
      float t8[8];
      t8_at(base, t8);
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += t8[j];
    }
  }
  // generate.rs:375-377: degenerate exit, no draw.
  if (!(sum > 0.0f) || !isfinite(sum)) {
    if (lane == 0) {
      store_result(a, b, id_at(0), len_b);
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }
  auto p_at = [&](uint32_t i) { return e_at(i) / sum; };  // generate.rs:378-380

  // generate.rs:384-395: longest prefix with p >= min_p * p_0, at least 1.
  uint32_t keep = n;
  if (P.min_p > 0.0f) {
    const float thr = P.min_p * p_at(0);
    for (uint32_t c = 0; c < n; c += 64u) {
      const uint32_t i = c + lane;
      const uint64_t fail = __ballot(i < n && !(p_at(i) >= thr));
      if (fail) {
        keep = c + (uint32_t)__ffsll((unsigned long long)fail) - 1u;
        break;
      }
    }
    if (keep < 1u) keep = 1u;
  }

  // generate.rs:397-411: the top-p fold over the kept prefix, in blocks of 8
  // (c never decreases); the deciding block is resolved one lane per term.
  uint32_t stop = keep;
  float total = 0.0f;
  {
    const float tp = P.top_p < 1.0f ? P.top_p : INFINITY;
    float c = 0.0f;
    bool hit_any = false;
    for (uint32_t w0 = 0; w0 < keep && !hit_any; w0 += cap) {
      const uint32_t cnt = stage(w0, keep, sum);
      float cprev = 0.0f;
      uint32_t k8 = 0u;
      bool brk = false;
      for (uint32_t base = 0; base < cnt; base += 8u) {
        float t8[8];
        t8_at(base, t8);
        cprev = c;
#pragma unroll
        for (int j = 0; j < 8; ++j) c += t8[j];
        k8 = base;
        if (c >= tp) {
          brk = true;
          break;
        }
      }
      if (brk) {
        float t8[8], t = cprev;
        t8_at(k8, t8);
#pragma unroll
        for (int j = 0; j < 8; ++j) t = (uint32_t)j <= lane ? t + t8[j] : t;
        const uint64_t hit = __ballot(lane < 8u && k8 + lane < cnt && t >= tp);
        const uint32_t h = (uint32_t)__ffsll((unsigned long long)hit);  // a hit exists: c >= tp
        stop = w0 + k8 + h;
        total = readlane_f32(t, h - 1u);
        hit_any = true;
      }
    }
    if (!hit_any) total = c;  // the padding adds +0.0
  }

  // generate.rs:412-419: r_0 = u * total; step i tests r_i < p_i, then
  // subtracts p_i; no hit picks the last kept term.
  const float u = next_f32(st);
  uint32_t pick = stop - 1u;
  {
    float r = u * total;
    bool found = false;
    for (uint32_t w0 = 0; w0 < stop && !found; w0 += cap) {
      const uint32_t cnt = stage(w0, stop, sum);
      float rprev = r;
      uint32_t k8 = 0u;
      bool neg = false;
      for (uint32_t base = 0; base < cnt; base += 8u) {
        float t8[8];
        t8_at(base, t8);
        rprev = r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r -= t8[j];
        k8 = base;
        if (r < 0.0f) {
          neg = true;
          break;
        }
      }
      if (neg) {
        float t8[8], t = rprev;
        t8_at(k8, t8);
#pragma unroll
        for (int j = 0; j < 8; ++j) t = (uint32_t)j < lane ? t - t8[j] : t;
        const float pj = lane < 8u ? buf[k8 + lane] : 0.0f;
        const uint64_t hit = __ballot(lane < 8u && k8 + lane < cnt && t < pj);
        if (hit) pick = w0 + k8 + (uint32_t)__ffsll((unsigned long long)hit) - 1u;
        found = true;
      }
    }
  }
  if (lane == 0) {
    store_result(a, b, id_at(pick), len_b);
    a.rng_state[b] = st;
    if (a.out_kept) a.out_kept[b] = stop;
  }
  if (a.out_probs) {
    float* prow = a.out_probs + (size_t)b * a.V;
    for (uint32_t i = lane; i < stop; i += 64u) prow[id_at(i)] = p_at(i);
  }
}

// Half an f32 ulp in the binade of x (x > 0; values below 2^-60 count as
// 2^-60), as an f64.
__device__ __forceinline__ double half_ulp_f32_at(double x) {
  const uint64_t bits = (uint64_t)__double_as_longlong(fmax(x, 0x1p-60));
  return __longlong_as_double((long long)((((bits >> 52) & 0x7ffull) - 24ull) << 52));
}

// The same computation for n <= 64 candidates held one per lane. The
// softmax sum runs as 64 dependent adds over terms broadcast through LDS
// (`buf`, 64 floats, 16-byte aligned); padding terms are +0.0, which leaves a
// sum of non-negative f32 terms unchanged. Top-p and the draw are decided from
// f64 prefix sums with error bounds, and the folds are replayed exactly only
// on a near tie (below).
__device__ __forceinline__ void draw_tail_bcast(const SampleArgs& a, uint32_t b, uint32_t len_b,
                                                const llmhip_params& P, uint32_t n, uint32_t my_key,
                                                uint32_t my_id, float u,
                                                uint64_t st_next, const uint64_t* tab, float* buf) {
  const uint32_t lane = lane_id();
  const bool act = lane < n;
  LLMHIP_TAIL_MARK(0);
  const uint32_t k0 = readlane_u32(my_key, 0);
  const float mx = k0 <= kKeyNaN ? -INFINITY : key2f(k0);
  const float e = act ? glibc_expf_tab(key2f(my_key) - mx, tab) : 0.0f;
  const float4* b4 = reinterpret_cast<const float4*>(buf);
  auto term4 = [](const float4& f, int i) __attribute__((always_inline)) {
    return i == 0 ? f.x : i == 1 ? f.y : i == 2 ? f.z : f.w;
  };

  // generate.rs:374: sum = ((0 + e_0) + e_1) + ... over the n terms, as 64
  // dependent adds: the terms past n are +0, which leave a sum >= e_0 = 1
  // (or a NaN one) unchanged. The terms come in four batches of 16, the
  // next batch loading while the current one is added.
  buf[lane] = e;
  float sum = 0.0f;
  {
    float4 wc[4], wn[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) wc[q] = b4[q];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      if (h < 3) {
#pragma unroll
        for (int q = 0; q < 4; ++q) wn[q] = b4[4 * (h + 1) + q];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sum += term4(wc[i >> 2], i & 3);
#pragma unroll
      for (int q = 0; q < 4; ++q) wc[q] = wn[q];
    }
  }
  LLMHIP_TAIL_MARK(1);
  // generate.rs:375-377: degenerate exit, no draw.
  if (__builtin_expect(!(sum > 0.0f) || !isfinite(sum), 0)) {
    if (lane == 0) {
      store_result(a, b, n > 0 ? my_id : 0u, len_b);
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }
  const float p = act ? e / sum : 0.0f;  // generate.rs:378-380

  // generate.rs:384-395: longest prefix with p >= min_p * p_0, at least 1.
  uint32_t keep = n;
  if (P.min_p > 0.0f) {
    const float thr = P.min_p * readlane_f32(p, 0);
    const uint64_t fail = __ballot(act && !(p >= thr));
    if (fail) keep = (uint32_t)__ffsll((unsigned long long)fail) - 1u;
    if (keep < 1u) keep = 1u;
  }

  // generate.rs:397-419 without the folds, where that is provably exact.
  // The top-p fold c_i = ((0 + p_0) + ...) + p_i and the walk r_0 = u*total,
  // r_{i+1} = r_i - p_i are f32 left folds. Each rounding is at most half
  // an f32 ulp (hulp) of its result. The c_k never decrease and are bounded
  // by the exact prefix sums P_i (an f64 wave scan): c_k <= c_i <=
  // P_i (1 + 2^-17) for k <= i, since |c_i - P_i| <= i 2^-24 P_i. So
  //   |c_i - P_i| <= B_i = i hulp(P_i (1 + 2^-17)),
  // and, while r_j >= p_j for j < i (then 0 <= r_j <= r_0),
  //   r_i in [u lo(c_s) - P_{i-1} - G_i, u hi(c_s) - P_{i-1} + G_i],
  //   G_i = (i + 1) hulp(u hi(c_s) (1 + 2^-16)),
  // with c_s the total at s = stop - 1 in [P_s - B_s, P_s + B_s]. Each
  // decision (c_i >= top_p, r_i < p_i) is taken from these intervals plus
  // an f64 rounding margin; the first decision that is true must be
  // certainly true and every one before it certainly false. Otherwise (a
  // near tie) the folds are replayed exactly.
  uint32_t stop = keep, pick = 0;
  bool cert = true;
  {
    const double pd = lane < keep ? (double)p : 0.0;
    const double Pi = wave_incl_scan_f64(pd);
    const double Bi = (double)lane * half_ulp_f32_at(Pi * (1.0 + 0x1p-17)) + 0x1p-45 * Pi;
    if (P.top_p < 1.0f) {
      const double tpd = (double)P.top_p;
      const uint64_t poss = __ballot(lane < keep && !(Pi + Bi < tpd));
      const uint64_t sure = __ballot(lane < keep && Pi - Bi >= tpd);
      if (poss) {
        const uint32_t i = (uint32_t)__ffsll((unsigned long long)poss) - 1u;
        if ((sure >> i) & 1ull) stop = i + 1u;
        else cert = false;
      }
    }
    if (cert) {
      const uint32_t s = stop - 1u;
      const double Ps = readlane_f64(Pi, s), Bs = readlane_f64(Bi, s), U = (double)u;
      const double lo0 = U * (Ps - Bs), hi0 = U * (Ps + Bs);
      const double Pprev = Pi - pd;  // P_{i-1}
      const double Gi = (double)(lane + 1u) * half_ulp_f32_at(hi0 * (1.0 + 0x1p-16)) + 0x1p-45 * (hi0 + Pprev);
      const double pdd = (double)p;
      const uint64_t poss = __ballot(lane < stop && !(lo0 - Pprev - Gi >= pdd));
      const uint64_t sure = __ballot(lane < stop && hi0 - Pprev + Gi < pdd);
      if (!poss) {
        pick = stop - 1u;
      } else {
        const uint32_t i = (uint32_t)__ffsll((unsigned long long)poss) - 1u;
        if ((sure >> i) & 1ull) pick = i;
        else cert = false;
      }
    }
  }

  LLMHIP_TAIL_MARK(2);
  if (__builtin_expect(!cert, 0)) {
    buf[lane] = p;
    // Terms 8k .. 8k+7, read from LDS per block (broadcast).
    auto block = [&](int kk, float (&t8)[8]) __attribute__((always_inline)) {
      const float4 lo = b4[2 * kk], hi = b4[2 * kk + 1];
      t8[0] = lo.x; t8[1] = lo.y; t8[2] = lo.z; t8[3] = lo.w;
      t8[4] = hi.x; t8[5] = hi.y; t8[6] = hi.z; t8[7] = hi.w;
    };

    // generate.rs:397-411: c_i = ((0 + p_0) + ...) + p_i; top-p keeps up to the
    // first c_i >= top_p (all when top_p >= 1 or never reached); the total
    // over the kept prefix is the fold at its last element. The fold runs in
    // blocks of 8 dependent adds; c never decreases (p_i >= 0), so only the
    // last value of a block is tested, and the block that holds the stop (or
    // the end of the kept prefix) is resolved once, after the loop: lane
    // 8k+j takes c_{8k+j} and one ballot finds the first c_i >= top_p.
    const float tp = P.top_p < 1.0f ? P.top_p : INFINITY;
    stop = keep;
    float total;
    {
      float c = 0.0f, cb[8];
      uint32_t k = 0;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        float t8[8];
        block(kk, t8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          c += t8[j];
          cb[j] = c;
        }
        k = (uint32_t)kk;
        if (c >= tp || 8u * (uint32_t)(kk + 1) >= keep) break;
      }
      const uint32_t k8 = 8u * k;
      float t = cb[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) t = lane == k8 + (uint32_t)j ? cb[j] : t;
      const uint64_t hit = __ballot(lane >= k8 && lane < k8 + 8u && lane < keep && t >= tp);
      if (hit) stop = (uint32_t)__ffsll((unsigned long long)hit);
      total = readlane_f32(t, stop - 1u);
    }

    // generate.rs:412-419: r_0 = u * total; step i tests r_i < p_i and then
    // subtracts p_i. r - p < 0 exactly when r < p (f32 denormals are kept), so
    // the block holding the pick is the first that ends negative; lane 8k+j
    // takes r_{8k+j} and compares it with its own p.
    pick = stop - 1u;
    {
      float r = u * total, rb[8];
      uint32_t k = 0;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        float t8[8];
        block(kk, t8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          rb[j] = r;
          r -= t8[j];
        }
        k = (uint32_t)kk;
        if (r < 0.0f || 8u * (uint32_t)(kk + 1) >= stop) break;
      }
      const uint32_t k8 = 8u * k;
      float t = rb[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) t = lane == k8 + (uint32_t)j ? rb[j] : t;
      const uint64_t hit = __ballot(lane >= k8 && lane < k8 + 8u && lane < stop && t < p);
      if (hit) pick = (uint32_t)__ffsll((unsigned long long)hit) - 1u;
    }
  }
  const uint32_t id = readlane_u32(my_id, pick);
  LLMHIP_TAIL_MARK(3);
  if (lane == 0) {
    store_result(a, b, id, len_b);
    a.rng_state[b] = st_next;
    if (a.out_kept) a.out_kept[b] = stop;
  }
  if (a.out_probs && lane < stop) a.out_probs[(size_t)b * a.V + my_id] = p;
}

}  // namespace llmhip
