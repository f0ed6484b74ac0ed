// Full-vocabulary rows (top_k == 0 or top_k >= V, temperature > 0) without
// sorting the row.
//
// crates/llm-core/src/generate.rs:364-419 sorts the whole row by (value
// desc, id asc) and then runs three f32 left folds in that order: the softmax
// sum (374), the top-p cumulative (397-409; its value at the cut is also the
// total of 411) and the inverse-CDF walk (412-419). This path produces the
// same results, bit for bit, from two facts:
//
//  * x = expf(w - max) is monotone in w (glibc's expf is monotone on
//    (-inf, 0]; checked exhaustively), and so is p = x / S. Each fold is
//    therefore a fold over a multiset of values taken in descending order.
//  * While a fold's running value F stays in one binade [2^E, 2^(E+1)),
//    fl(F + t) = F + rne(t / u) * u with u = 2^(E-23): an integer count of
//    ulps that does not depend on where t comes in the order, except at an
//    exact half-ulp tie, where round-half-even looks at the parity of F.
//
// The row is bucketed by y = w - max, 128 buckets per unit of y (bucket 0
// holds the max). An approximate prefix of the buckets' masses shows which
// buckets may hold a binade crossing or a stop (the top-p cut, the walk's
// pick). Those "zones" are gathered into LDS, sorted, and replayed 64
// elements at a time in integer ulps, with the elements where something
// happens (a crossing, a stop, a tie) stepped in f32. Every other
// ("certain") bucket adds its exact integer ulp count with LDS atomics, and
// the certain runs between zones are added as integers. A certain bucket
// that holds a tie is split at the tie: a second sweep sums the ulp counts of
// the bucket's elements that come before each tie, and the replay applies
// round-half-even to the tie with the parity it then knows.
//
// The softmax sum runs alone (the other folds need S). The top-p cumulative
// and the walk run together: one classification word per bucket for both,
// one exact pass, one tie split and one zone sort, then the two replays one
// after the other (the walk is classified for every start its total allows).
//
// Every assumption the approximate prefix made is checked exactly during the
// replay; a row whose check fails, or that needs more zones than the LDS
// holds, is handed to the sorting path (general_row), so the ids are the
// reference's either way.
//
// Each pass streams the row again (the re-reads of a row that a CU has just
// read come from the MALL).
#pragma once
#include "draw_tail.h"
#include "fast_row.h"
#include "sampler_common.h"
#include "wave_ops.h"

namespace llmhip {

constexpr uint32_t kVB = 4096;             // buckets
constexpr float kVR = 128.0f;              // buckets per unit of y
constexpr uint32_t kVZones = 320;          // zones (of either fold)
constexpr uint32_t kVZoneEls = 4096;       // gathered elements (of either fold)
constexpr uint32_t kVTies = 256;           // ties in certain buckets (of either fold)
constexpr uint32_t kVHash = 2048;          // repetition-count table slots
constexpr uint32_t kVMaxDistinct = 1536;   // distinct history ids the table takes
constexpr uint32_t kVBits = 4096;          // words of the history filter (bit id mod 2^17)
constexpr uint32_t kVListCap = 65536;      // min-p candidates listed per row
constexpr uint32_t kHashEmpty = 0xffffffffu;
constexpr int32_t kNoE = -1000;            // segment without certain buckets
constexpr uint32_t kNoPos = 0xffffffffu;

enum : uint8_t { kBSkip = 0, kBCert = 1, kBZone = 2, kBTie = 3 };

// misc[] slots
enum : uint32_t {
  kVFail = 0,        // nonzero: hand the row to general_row
  kVBeyond0 = 1,     // first bucket certain to lie past fold 0's stop
  kVBeyond1 = 2,     // the same for fold 1
  kVStopZone = 3,    // first bucket that may hold fold 0's stop
  kVNTies = 4,       // ties found in certain buckets
  kVCount = 5,       // terms >= the min-p threshold
  kVDistinct = 6,    // distinct history ids
  kVCand = 7,        // min-p candidates listed
  kVSplitDone = 8,   // waves done with the tie split
  kVKeep = 9,        // the walk's end (sorted positions kept)
  kVRes = 10,        // fold results, 4 words per fold
  kVTieMax = 18,     // last bucket holding a tie
  kVSortDone = 19,   // waves done with their share of the zone sort
  kVSplitNext = 20,  // next block of the tie split to claim
  kVMisc = 21,
};

struct VocabLds {
  uint32_t cnt[kVB];   // elements per bucket
  float asum[kVB];     // approximate sum of x per bucket; then fold 1's ulp counts
  uint32_t D[kVB];     // exact ulp counts of fold 0's certain buckets
  uint32_t binfo[kVB];  // per bucket: slot, both folds' classes and binades (bpack)
  // Zones (buckets gathered or split at ties, for either fold) in bucket
  // order; segment z of a fold holds its certain buckets before zone z.
  uint32_t zb[kVZones];
  uint32_t zbase[kVZones + 1];
  uint32_t zcur[kVZones];
  uint32_t zpos[kVZones];       // sorted position of the zone bucket's first element
  uint16_t zt0[2][kVZones];     // tie zones: a fold's first tie (sorted tie order), count
  uint16_t ztn[2][kVZones];
  unsigned long long seg[2][kVZones + 1];
  int32_t segE[2][kVZones + 1];
  uint32_t segTub[kVZones + 1];  // the walk: largest term bound of the segment
  // Gathered zone elements, packed as key << 32 | ~id so that a larger value
  // comes first in the reference's order; after the sort, term << 32 | ~id.
  // zperm[base + r] is the element at sorted position r of its zone. Before
  // the first fold, zpk holds the buckets' masses (amass).
  unsigned long long zpk[kVZoneEls];
  uint16_t zperm[kVZoneEls];
  // Ties in certain buckets: key, id, ulp count, fold << 31 | bucket; ulp sum
  // above each.
  uint32_t tkey[kVTies], tidx[kVTies], tq[kVTies], tbk[kVTies], tab[kVTies];
  uint16_t tord[kVTies];
  uint32_t hkey[kVHash];
  float hval[kVHash];
  uint32_t hbits[kVBits];  // set for every history id (mod 32 * kVBits): the table is probed only then
  double scand[kWaves];
  double amix;             // approximate mass of the bucket the min-p threshold splits
  uint32_t scanu[kWaves];
  float redf[kWaves];
  uint32_t misc[kVMisc];
  uint64_t exptab[32];
};

// A bucket's word: slot (bits 0-8: zone slot, or segment index for certain
// buckets), fold 0's class (9-10), fold 1's class (11-12), step bits (13-14),
// fold 0's binade + 128 (16-23), fold 1's binade + 128 (24-31). Step bit f:
// the bucket is gathered and certain for fold f, but holds a tie for it, so
// fold f replays it element by element rather than adding its ulp count.
static_assert(kVZones < 512, "slot bits");
constexpr uint32_t kBStep = 1u << 13;
__device__ __forceinline__ uint32_t bpack(uint32_t slot, uint32_t c0, uint32_t c1, int e0, int e1) {
  return slot | (c0 << 9) | (c1 << 11) | ((uint32_t)(e0 + 128) << 16) | ((uint32_t)(e1 + 128) << 24);
}
__device__ __forceinline__ uint32_t bcls_shift(int f) { return 9u + 2u * (uint32_t)f; }
__device__ __forceinline__ uint32_t bcls(uint32_t bi, int f) { return (bi >> bcls_shift(f)) & 3u; }
__device__ __forceinline__ uint32_t bslot(uint32_t bi) { return bi & 511u; }
__device__ __forceinline__ int bbin(uint32_t bi, int f) { return (int)((bi >> (16 + 8 * f)) & 255u) - 128; }

__device__ __forceinline__ uint32_t vbucket(float y) {
  const float ny = -y;
  return ny < 32.0f ? (uint32_t)(ny * kVR) : kVB - 1u;
}

// Binade of a positive normal double.
__device__ __forceinline__ int dbinade(double v) {
  return (int)((uint64_t)(__double_as_longlong(v) >> 52) & 0x7ffu) - 1023;
}

__device__ __forceinline__ float from_units(uint32_t M, int E) {
  return __uint_as_float(((uint32_t)(E + 127) << 23) | (M & 0x7fffffu));
}

// t >= 0 in units of 2^(E-23), rounded to nearest; tie: exactly half-way
// (the result is then the lower neighbour). big: t >= 2^E, which a certain
// bucket never holds.
__device__ __forceinline__ uint32_t rne_units(float t, int E, bool& tie, bool& big) {
  const uint32_t u = __float_as_uint(t);
  const uint32_t ef = (u >> 23) & 255u;
  const uint32_t m = ef ? ((u & 0x7fffffu) | 0x800000u) : (u & 0x7fffffu);
  const int s = E - (ef ? (int)ef - 127 : -126);
  tie = false;
  big = s <= 0;
  if (s <= 0 || s >= 25) return 0u;
  const uint32_t q = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1);
  tie = rem == half;
  return q + (rem > half ? 1u : 0u);
}

// Exclusive prefix over the workgroup; total gets the sum. All threads call.
__device__ __forceinline__ uint32_t block_scan_u32(uint32_t x, uint32_t* tmp, uint32_t& total) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t inc = wave_incl_scan(x);
  if (lane == 63u) tmp[wave] = inc;
  __syncthreads();
  const uint32_t wv = lane < kWaves ? tmp[lane] : 0u;
  const uint32_t winc = wave_incl_scan(wv);
  total = readlane_u32(winc, kWaves - 1u);
  const uint32_t base = readlane_u32(winc - wv, wave);
  __syncthreads();
  return base + inc - x;
}
__device__ __forceinline__ double block_scan_f64(double x, double* tmp, double& total) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const double inc = wave_incl_scan_f64(x);
  if (lane == 63u) tmp[wave] = inc;
  __syncthreads();
  const double wv = lane < kWaves ? tmp[lane] : 0.0;
  const double winc = wave_incl_scan_f64(wv);
  total = readlane_f64(winc, kWaves - 1u);
  const double base = readlane_f64(winc - wv, wave);
  __syncthreads();
  return base + (inc - x);
}

// Element source: for_each(f) calls f(w, id) once for every element of the
// row, w being the masked, penalized logit divided by the temperature.
// Row streamed from memory by every pass: float4 groups, two batches of 4
// per thread in flight (the next batch loads while this one is visited), or
// scalars when the row is not 16-byte aligned.
//
// VP gives an element's value in parts: pre(i, v) the allowed mask, pen()
// whether the row has penalized history ids, hit(i) / hit4(i) their filter
// bits, hist(i, v) the penalized value of a history id (v when i is not
// one), post(v) the division by T. History ids are about 1% of a row, but a
// wave looking one up at every element position where one of its lanes
// holds one would look up at almost every position: each lane's history
// ids among its 16 elements are looked up one at a time instead (finish).
template <class VP>
struct StreamSrc {
  const float* row;
  uint32_t V;
  bool vec4;
  VP vp;
  // Element i's value from its logit v.
  __device__ __forceinline__ float value(uint32_t i, float v) const {
    v = vp.pre(i, v);
    if (vp.pen() && vp.hit(i)) v = vp.hist(i, v);
    return vp.post(v);
  }
  // w holds pre() of the lane's 16 elements (ids id_of(e)); hm marks the
  // history ids among them. Their values are replaced, then post() applied
  // to every valid element.
  template <class IdOf>
  __device__ __forceinline__ void finish(float (&w)[16], uint32_t valid, uint32_t hm, IdOf&& id_of) const {
    while (hm != 0u) {
      const uint32_t e = (uint32_t)__builtin_ctz(hm);
      hm &= hm - 1u;
      float we = w[0];
#pragma unroll
      for (int q = 1; q < 16; ++q) we = e == (uint32_t)q ? w[q] : we;
      we = vp.hist(id_of(e), we);
#pragma unroll
      for (int q = 0; q < 16; ++q) w[q] = e == (uint32_t)q ? we : w[q];
    }
#pragma unroll
    for (int q = 0; q < 16; ++q)
      if ((valid >> q) & 1u) w[q] = vp.post(w[q]);
  }
  // Elements 4 * (q0 + t + kBlock * s) + c of float4 groups cur[s], s < 4:
  // their pre() values, validity and history marks.
  __device__ __forceinline__ void pre_quads(const float4 (&v4)[4], uint32_t base, uint32_t stride, float (&w)[16],
                                            uint32_t& valid, uint32_t& hm) const {
    valid = 0u;
    hm = 0u;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t i = 4u * (base + stride * (uint32_t)s);
      const float v[4] = {v4[s].x, v4[s].y, v4[s].z, v4[s].w};
      const uint32_t hb = vp.pen() ? vp.hit4(i) : 0u;  // one filter word holds the four ids
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bool in = i + c < V;
        w[4 * s + c] = in ? vp.pre(i + c, v[c]) : 0.0f;
        valid |= (in ? 1u : 0u) << (4 * s + c);
        hm |= (in && ((hb >> c) & 1u) ? 1u : 0u) << (4 * s + c);
      }
    }
  }
  template <class F>
  __device__ __forceinline__ void for_each(F&& f) const {
    const uint32_t t = threadIdx.x;
    constexpr uint32_t nt = kBlock;
    if (!vp.pen()) {
      // No history ids: each element's value as it is visited.
      if (vec4) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
        const uint32_t nq = (V + 3u) / 4u;
        float4 cur[4], nxt[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint32_t q = t + nt * s;
          cur[s] = q < nq ? r4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        for (uint32_t q0 = 0; q0 < nq; q0 += 4u * nt) {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const uint32_t q = q0 + 4u * nt + t + nt * s;
            nxt[s] = q < nq ? r4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const uint32_t i = 4u * (q0 + t + nt * s);
            const float v[4] = {cur[s].x, cur[s].y, cur[s].z, cur[s].w};
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (i + c < V) f(vp.post(vp.pre(i + c, v[c])), i + c);
          }
#pragma unroll
          for (int s = 0; s < 4; ++s) cur[s] = nxt[s];
        }
      } else {
        uint32_t i = t;
        for (; i + 7u * nt < V; i += 8u * nt) {
          float v[8];
#pragma unroll
          for (int s = 0; s < 8; ++s) v[s] = row[i + nt * s];
#pragma unroll
          for (int s = 0; s < 8; ++s) f(vp.post(vp.pre(i + nt * s, v[s])), i + nt * s);
        }
        for (; i < V; i += nt) f(vp.post(vp.pre(i, row[i])), i);
      }
      return;
    }
    float w[16];
    uint32_t valid, hm;
    if (vec4) {
      const float4* r4 = reinterpret_cast<const float4*>(row);
      const uint32_t nq = (V + 3u) / 4u;
      float4 cur[4], nxt[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t q = t + nt * s;
        cur[s] = q < nq ? r4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      for (uint32_t q0 = 0; q0 < nq; q0 += 4u * nt) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint32_t q = q0 + 4u * nt + t + nt * s;
          nxt[s] = q < nq ? r4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        pre_quads(cur, q0 + t, nt, w, valid, hm);
        finish(w, valid, hm, [&](uint32_t e) { return 4u * (q0 + t + nt * (e >> 2)) + (e & 3u); });
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if ((valid >> e) & 1u) f(w[e], 4u * (q0 + t + nt * (uint32_t)(e >> 2)) + (uint32_t)(e & 3));
#pragma unroll
        for (int s = 0; s < 4; ++s) cur[s] = nxt[s];
      }
    } else {
      for (uint32_t i0 = t; i0 < V; i0 += 16u * nt) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t i = i0 + nt * e;
          w[e] = i < V ? row[i] : 0.0f;
        }
        valid = 0u;
        hm = 0u;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t i = i0 + nt * e;
          const bool in = i < V;
          w[e] = in ? vp.pre(i, w[e]) : 0.0f;
          valid |= (in ? 1u : 0u) << e;
          hm |= (in && vp.pen() && vp.hit(i) ? 1u : 0u) << e;
        }
        finish(w, valid, hm, [&](uint32_t e) { return i0 + nt * e; });
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if ((valid >> e) & 1u) f(w[e], i0 + nt * (uint32_t)e);
      }
    }
  }
  // Element i's post-temperature value.
  __device__ __forceinline__ float value_at(uint32_t i) const { return value(i, row[i]); }
  // Blocks of 1024 elements (a wave takes one at a time: load_block).
  __device__ __forceinline__ uint32_t blocks() const { return (V + 1023u) / 1024u; }
  // The calling lane's elements of block blk (16 of its 1024: the wave
  // takes the block): values w, ids, and bit e of valid set for each that
  // exists.
  __device__ __forceinline__ void load_block(uint32_t blk, float (&w)[16], uint32_t (&id)[16], uint32_t& valid) const {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t hm;
    if (vec4) {
      const float4* r4 = reinterpret_cast<const float4*>(row);
      const uint32_t nq = (V + 3u) / 4u;
      float4 v4[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t q = blk * 256u + lane + 64u * s;
        v4[s] = q < nq ? r4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) id[e] = 4u * (blk * 256u + lane + 64u * (uint32_t)(e >> 2)) + (uint32_t)(e & 3);
      if (!vp.pen()) {
        valid = 0u;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float v[4] = {v4[s].x, v4[s].y, v4[s].z, v4[s].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const bool in = id[4 * s + c] < V;
            w[4 * s + c] = in ? vp.post(vp.pre(id[4 * s + c], v[c])) : 0.0f;
            valid |= (in ? 1u : 0u) << (4 * s + c);
          }
        }
        return;
      }
      pre_quads(v4, blk * 256u + lane, 64u, w, valid, hm);
      finish(w, valid, hm, [&](uint32_t e) { return 4u * (blk * 256u + lane + 64u * (e >> 2)) + (e & 3u); });
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t i = blk * 1024u + lane + 64u * e;
        w[e] = i < V ? row[i] : 0.0f;
      }
      valid = 0u;
      hm = 0u;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t i = blk * 1024u + lane + 64u * e;
        const bool in = i < V;
        w[e] = in ? vp.pre(i, w[e]) : 0.0f;
        id[e] = i;
        valid |= (in ? 1u : 0u) << e;
        hm |= (in && vp.pen() && vp.hit(i) ? 1u : 0u) << e;
      }
      finish(w, valid, hm, [&](uint32_t e) { return blk * 1024u + lane + 64u * e; });
    }
  }
};

// The min-p candidates of a row, listed by the histogram pass as (key, id)
// pairs in the row's scratch: once S is known, the top-p and walk folds read
// only these when every bucket that can pass min-p was listed.
struct ListSrc {
  const uint2* list;
  uint32_t n;
  template <class F>
  __device__ __forceinline__ void for_each_part(F&& f, uint32_t t0, uint32_t nt) const {
    for (uint32_t j = threadIdx.x - t0; j < n; j += nt) {
      const uint2 e = list[j];
      f(key2f(e.x), e.y);
    }
  }
  template <class F>
  __device__ __forceinline__ void for_each(F&& f) const {
    for_each_part(f, 0u, kBlock);
  }
  __device__ __forceinline__ uint32_t blocks() const { return (n + 1023u) / 1024u; }
  __device__ __forceinline__ void load_block(uint32_t blk, float (&w)[16], uint32_t (&id)[16], uint32_t& valid) const {
    const uint32_t lane = threadIdx.x & 63u;
    valid = 0u;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const uint32_t j = blk * 1024u + lane + 64u * s;
      const uint2 e = j < n ? list[j] : make_uint2(0u, 0u);
      w[s] = key2f(e.x);
      id[s] = e.y;
      valid |= (j < n ? 1u : 0u) << s;
    }
  }
};

// exp(y) for -80 <= y <= 0 from the hardware exp2: y * log2(e) = k + f with
// the product split exactly by an FMA, |f| <= 1/2, and v_exp_f32, whose
// relative error on [-1/2, 1/2] is at most 1.4 * 2^-24 (measured over every
// input). The result is within 2^-22 of glibc's expf (which is itself within
// 0.502 ulp of exp). Used only to settle decisions that have that much room.
__device__ __forceinline__ float cheap_x(float y) {
  const float L1 = 0x1.715476p+0f, L2 = 0x1.4ae0bep-26f;  // log2(e) = L1 + L2 + O(2^-50)
  const float hi = y * L1;
  const float lo = __builtin_fmaf(y, L1, -hi) + y * L2;
  const float kf = rintf(hi);
  const float f = (hi - kf) + lo;  // hi - kf is exact
  return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(f), (int)kf);
}

// One or two folds over the row's terms in sorted order (see the file
// comment). Two folds (the top-p cumulative and the walk, which take the same
// terms) share the classification's layout, the exact pass, the tie split and
// the zone sort; only their replays are separate.
struct FoldSpec {
  float F0;          // starting value (the walk: set by run_folds)
  float S;           // terms are x / S (0: the terms are x)
  float thr;         // terms below thr are outside the fold (min-p); <= 0: none
  float stop_ge;     // add folds: stop at the first F >= stop_ge
  bool sub;          // the walk: stop before t when F < t, else F -= t
};

struct FoldRes {
  float F;
  uint32_t stop_pos;  // kNoPos: no stop
  uint32_t stop_id;
  uint32_t stop_bk;
};

// (key desc, id asc): the reference's order (generate.rs:364-367).
__device__ __forceinline__ bool before(uint32_t ka, uint32_t ia, uint32_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// NF == 1: fs[0] only. NF == 2: fs[0] is the top-p cumulative and fs[1] the
// walk; the walk's start is u * (fold 0's result), and while the two are
// classified it is only known to lie in an interval, which the walk's margin
// covers. The walk ends at sorted position keep (returned in keep_out): fold
// 0's cut + 1, or without a cut the number of terms >= thr (at least 1) when
// keep_count, else keep_default.
//
// tl lists every element of buckets 0 .. tl_k when tl_ok; a tie split whose
// ties all lie in those buckets reads it instead of src.
template <int NF, class Src>
__device__ __forceinline__ bool run_folds(FoldSpec (&fs)[NF], float mx, float u, uint32_t keep_default, bool keep_count,
                                          VocabLds& L, const Src& src, const ListSrc& tl, bool tl_ok, uint32_t tl_k,
                                          FoldRes (&res)[NF], uint32_t& keep_out, const SampleArgs& a) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t k0 = tid * 4u;
  const float S = fs[0].S, thr = fs[0].thr;  // the same terms for both folds
  const double scale = S > 0.0f ? 1.0 / (double)S : 1.0;
  auto term_of = [&](float x) __attribute__((always_inline)) { return S > 0.0f ? x / S : x; };
  // Fold 1's exact ulp counts live where the approximate masses were: those
  // are no longer needed once both folds are classified.
  uint32_t* Dw = reinterpret_cast<uint32_t*>(L.asum);
  auto Df = [&](int f) __attribute__((always_inline)) -> uint32_t* { return f == 0 ? L.D : Dw; };

  for (uint32_t s = tid; s <= kVZones; s += kBlock) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      L.seg[f][s] = 0ull;
      L.segE[f][s] = kNoE;
    }
    L.segTub[s] = 0u;
  }
  if (tid == 0) {
    L.amix = 0.0;
    L.misc[kVBeyond0] = kVB;
    L.misc[kVBeyond1] = kVB;
    L.misc[kVStopZone] = kVB;
    L.misc[kVNTies] = 0u;
    L.misc[kVCount] = 0u;
    L.misc[kVSplitDone] = 0u;
    L.misc[kVTieMax] = 0u;
    L.misc[kVSortDone] = 0u;
    L.misc[kVSplitNext] = 0u;
  }

  // Classification of this thread's 4 buckets from the approximate prefix.
  // The margin is 6 sigma of a random walk of half-ulp rounding errors plus
  // 2^-20 of the value for the approximate masses; the replay checks every
  // consequence exactly, so a wrong guess costs a hand-over, not an id.
  uint32_t c4[4];
  double a4[4];
  float tub4[4], tlb4[4];
  uint8_t cl[2][4];
  int e4[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
  uint32_t cs = 0;
  double as = 0.0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t k = k0 + j;
    c4[j] = L.cnt[k];
    tub4[j] = term_of(glibc_expf_tab(-(float)k / kVR, L.exptab));
    tlb4[j] = k + 1 < kVB ? term_of(glibc_expf_tab(-(float)(k + 1) / kVR, L.exptab)) : 0.0f;
    const bool out = !c4[j] || (thr > 0.0f && tub4[j] < thr);
    a4[j] = out ? 0.0 : (double)L.asum[k] * scale;
#pragma unroll
    for (int f = 0; f < 2; ++f) cl[f][j] = (out || f >= NF) ? kBSkip : kBCert;
    cs += c4[j];
    as += a4[j];
  }
  uint32_t ctot;
  const uint32_t cpre = block_scan_u32(cs, L.scanu, ctot);
  double atot;
  const double apre = block_scan_f64(as, L.scand, atot);
  // The one bucket that the min-p threshold splits: its mass counts in full
  // above, but only part of it is in the folds.
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (a4[j] > 0.0 && thr > 0.0f && tlb4[j] < thr) L.amix = a4[j];
  // One fold's classes for this thread's buckets. kend: buckets from there
  // on are outside the fold. err0: a margin added to every interval.
  auto classify = [&](int f, const FoldSpec& sp, uint32_t kend, double err0, uint32_t beyond_slot)
      __attribute__((always_inline)) {
    const double sg = sp.sub ? -1.0 : 1.0;
    uint32_t nb = cpre;
    double P = apre;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t k = k0 + j;
      const double Ga = sp.F0 + sg * P, Gb = sp.F0 + sg * (P + a4[j]);
      if (k >= kend) cl[f][j] = kBSkip;
      if (cl[f][j] != kBSkip) {
        // Bucket 0 and the bucket that the min-p threshold splits are always
        // gathered.
        const bool forced = k == 0 || (thr > 0.0f && tlb4[j] < thr);
        double hi = fmax(Ga, Gb), lo = fmin(Ga, Gb);
        const double err = (6.0 * sqrt((double)nb + 1.0) * 0x1p-24 + 0x1p-20) * (sp.sub ? (double)sp.F0 : hi) + err0;
        if (!forced && ((!sp.sub && Ga - err >= (double)sp.stop_ge) || (sp.sub && Ga + err < 0.0))) {
          cl[f][j] = kBSkip;
          atomicMin(&L.misc[beyond_slot], k);
        } else {
          lo -= err;
          hi += err;
          const bool stopz = !sp.sub && hi >= (double)sp.stop_ge;
          if (stopz && f == 0) atomicMin(&L.misc[kVStopZone], k);  // the cut can first fall here
          const int E = lo > 0.0 ? dbinade(lo) : 0;
          if (forced || stopz || !(lo > 0.0) || E != dbinade(hi) || E < -120 || E > 120 ||
              (sp.sub && lo <= (double)tub4[j] * (1.0 + 0x1p-20))) {
            cl[f][j] = kBZone;
          } else {
            e4[f][j] = E;
          }
        }
      }
      nb += c4[j];
      P += a4[j];
    }
  };
  classify(0, fs[0], kVB, 0.0, kVBeyond0);
  __syncthreads();
  LLMHIP_MARK(NF == 1 ? 3 : 7);
  const uint32_t kb0 = L.misc[kVBeyond0];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (k0 + j >= kb0) cl[0][j] = kBSkip;
  uint32_t kb1 = kVB;
  if constexpr (NF == 2) {
    // The walk starts at u * total, total being fold 0's value where it ends.
    // At a cut, total lies in [stop_ge, stop_ge + the largest term of the
    // first bucket that can hold the cut]; without one, it is the sum of all
    // the fold's terms, which the approximate masses bound. The walk is
    // classified for any start in that range (its margin covers the range);
    // the replay then starts from the exact value and checks everything.
    const uint32_t ksz = L.misc[kVStopZone];
    const double stop_ge = (double)fs[0].stop_ge;
    double tlo = INFINITY, thi = -INFINITY;
    if (ksz < kVB) {
      const double tmax = (double)term_of(glibc_expf_tab(-(float)ksz / kVR, L.exptab));
      tlo = stop_ge;
      thi = stop_ge + tmax * (1.0 + 0x1p-20) + stop_ge * 0x1p-23;
    }
    const double e = (6.0 * sqrt((double)ctot + 1.0) * 0x1p-24 + 0x1p-20) * atot;
    if (!(atot - L.amix - e >= stop_ge)) {  // the fold may end without a cut
      tlo = fmin(tlo, atot - L.amix - e);
      thi = fmax(thi, fmin(atot + e, stop_ge));
    }
    if (!(tlo <= thi) || !(thi < 0x1p100)) return false;
    const double r0_lo = (double)u * tlo * (1.0 - 0x1p-22), r0_hi = (double)u * thi * (1.0 + 0x1p-22);
    fs[1].F0 = (float)(0.5 * (r0_lo + r0_hi));
    classify(1, fs[1], kb0, 0.5 * (r0_hi - r0_lo) + (double)fs[1].F0 * 0x1p-23, kVBeyond1);
    __syncthreads();
    kb1 = L.misc[kVBeyond1];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (k0 + j >= kb1) cl[1][j] = kBSkip;
  }

  // Zone slots, segment indices and element bases, in bucket order. A bucket
  // is a gathering zone when it is a zone for either fold, a tie zone when it
  // holds a tie of either fold, and otherwise belongs to the segment before
  // the next zone. Run a second time when ties turned certain buckets into
  // tie zones: those hold no elements, so every gathering zone keeps its
  // element base, and its gathered count and step bits are carried over.
  uint32_t nz = 0;
  uint32_t carry4[4] = {0u, 0u, 0u, 0u};  // a gathering bucket's count and step bits, across a re-layout
  auto gathers = [&](int j) __attribute__((always_inline)) { return cl[0][j] == kBZone || cl[1][j] == kBZone; };
  auto ties_in = [&](int j) __attribute__((always_inline)) { return cl[0][j] == kBTie || cl[1][j] == kBTie; };
  auto layout = [&]() __attribute__((always_inline)) -> bool {
    uint32_t zc = 0, ze = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      zc += (gathers(j) || ties_in(j)) ? 1u : 0u;
      ze += gathers(j) ? c4[j] : 0u;
    }
    uint32_t nel;
    uint32_t zi = block_scan_u32(zc, L.scanu, nz);
    uint32_t ei = block_scan_u32(ze, L.scanu, nel);
    if (nz > kVZones || nel > kVZoneEls) return false;
    uint32_t pos = cpre;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t k = k0 + j;
      const bool zone = gathers(j) || ties_in(j);
      L.binfo[k] = bpack(zi, cl[0][j], cl[1][j], e4[0][j], e4[1][j]) | (carry4[j] & (kBStep * 3u));
      if (zone) {
        L.zb[zi] = k;
        L.zbase[zi] = ei;
        L.zcur[zi] = carry4[j] & (kBStep - 1u);
        L.zpos[zi] = pos;
        ++zi;
        if (gathers(j)) ei += c4[j];
      } else {
#pragma unroll
        for (int f = 0; f < NF; ++f)
          if (cl[f][j] == kBCert) {
            L.segE[f][zi] = e4[f][j];
            if (fs[f].sub) atomicMax(&L.segTub[zi], __float_as_uint(tub4[j]));
          }
      }
      pos += c4[j];
    }
    if (tid == 0) L.zbase[nz] = nel;
    return true;
  };
  if (!layout()) return false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    L.D[k0 + j] = 0u;
    if constexpr (NF == 2) Dw[k0 + j] = 0u;
  }
  __syncthreads();

  // Exact pass: certain buckets add ulp counts, zones gather, ties are listed.
  // A term is first taken from a cheap exp (cheap_x: within 2^-22 of glibc's
  // expf, and after the reciprocal multiply within 2^-20 of the exact term);
  // the exact term is computed only when the cheap one cannot settle the
  // min-p test or an ulp count (a scaled value within value * 2^-20 of a
  // half-integer, or a term near the binade).
  const float rcpS = S > 0.0f ? 1.0f / S : 1.0f;
  uint32_t nin = 0;
  src.for_each([&](float w, uint32_t i) __attribute__((always_inline)) {
    const float y = w - mx;
    const uint32_t k = vbucket(y);
    const uint32_t bi = L.binfo[k];
    // The cheap term is computed while the bucket's word is read (the
    // empty asm keeps it ahead of the class test that waits for the read).
    const bool cheap = y >= -80.0f;
    float ta = cheap ? cheap_x(y) * rcpS : 0.0f;
    asm volatile("" : "+v"(ta));
    const uint32_t c0 = bcls(bi, 0), c1 = bcls(bi, 1);
    if (c0 == kBSkip && c1 == kBSkip) return;
    float t = -1.0f;  // the exact term, once computed
    if (thr > 0.0f) {
      bool in;
      if (cheap && ta >= thr * (1.0f + 0x1p-19f)) {
        in = true;
      } else if (cheap && ta < thr * (1.0f - 0x1p-19f)) {
        in = false;
      } else {
        t = term_of(glibc_expf_tab(y, L.exptab));
        in = t >= thr;
      }
      if (!in) return;
    }
    if (c0 != kBSkip) ++nin;
    // A gathered bucket that is certain for the other fold is also counted
    // for it, so that fold adds it as one integer.
    const bool gath = c0 == kBZone || c1 == kBZone;
    if (gath) {
      const uint32_t z = bslot(bi);
      const uint32_t e = L.zbase[z] + atomicAdd(&L.zcur[z], 1u);
      L.zpk[e] = ((unsigned long long)f2key(w) << 32) | (uint32_t)~i;
      if constexpr (NF == 1) return;
    }
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if ((f == 0 ? c0 : c1) != kBCert) continue;
      const int E = bbin(bi, f);
      if (cheap && t < 0.0f) {
        const float v = __builtin_amdgcn_ldexpf(ta, 23 - E);  // ta in units of 2^(E-23), exactly
        if (v < 0x1p22f) {
          const float fl = floorf(v), fr = v - fl;
          if (fabsf(fr - 0.5f) > v * 0x1p-20f + 0x1p-40f) {
            atomicAdd(&Df(f)[k], (uint32_t)fl + (fr > 0.5f ? 1u : 0u));
            continue;
          }
        }
      }
      if (t < 0.0f) t = term_of(glibc_expf_tab(y, L.exptab));
      bool tie, big;
      const uint32_t q = rne_units(t, E, tie, big);
      if (gath && (tie || big)) {
        atomicOr(&L.binfo[k], kBStep << f);  // this fold replays the bucket element by element
        continue;
      }
      if (big) L.misc[kVFail] = 1u;
      if (tie) {
        const uint32_t s = atomicAdd(&L.misc[kVNTies], 1u);
        if (s < kVTies) {
          L.tkey[s] = f2key(w);
          L.tidx[s] = i;
          L.tq[s] = q;
          L.tbk[s] = k | ((uint32_t)f << 31);
          L.tab[s] = 0u;
        }
      } else {
        atomicAdd(&Df(f)[k], q);
      }
    }
  });
  nin = wave_sum(nin);
  if (lane == 0) atomicAdd(&L.misc[kVCount], nin);
  __syncthreads();
  LLMHIP_MARK(NF == 1 ? 4 : 8);
  const uint32_t nt = L.misc[kVNTies];
  if (L.misc[kVFail] || nt > kVTies) return false;

  if (nt) {
    // Ties in certain buckets: sort them by (fold, bucket, key desc, id asc),
    // make their buckets tie zones of their fold, and (below) sum each
    // bucket's ulp counts above each tie.
    for (uint32_t s = tid; s < nt; s += kBlock) {
      uint32_t r = 0;
      const uint32_t bs = L.tbk[s], ks = L.tkey[s], is = L.tidx[s];
      for (uint32_t v = 0; v < nt; ++v) {
        const uint32_t bu = L.tbk[v];
        r += (bu < bs || (bu == bs && before(L.tkey[v], L.tidx[v], ks, is))) ? 1u : 0u;
      }
      L.tord[r] = (uint16_t)s;
      atomicMax(&L.misc[kVTieMax], bs & 0x7fffffffu);
      const uint32_t f = bs >> 31;
      atomicOr(&L.binfo[bs & 0x7fffffffu], (uint32_t)(kBTie ^ kBCert) << bcls_shift(f));  // CERT -> TIE
    }
    for (uint32_t s = tid; s <= kVZones; s += kBlock) {
#pragma unroll
      for (int f = 0; f < 2; ++f) L.segE[f][s] = kNoE;
      L.segTub[s] = 0u;
    }
    __syncthreads();
    // The buckets' state comes back from LDS (with the ties' classes), so
    // none of it stays in registers across the exact pass.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t k = k0 + j;
      const uint32_t bi = L.binfo[k];
      c4[j] = L.cnt[k];
      tub4[j] = term_of(glibc_expf_tab(-(float)k / kVR, L.exptab));
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        cl[f][j] = (uint8_t)bcls(bi, f);
        e4[f][j] = bbin(bi, f);
      }
      carry4[j] = gathers(j) ? L.zcur[bslot(bi)] | (bi & (kBStep * 3u)) : 0u;
    }
    if (!layout()) return false;
    __syncthreads();
    for (uint32_t z = tid; z < nz; z += kBlock) {
      const uint32_t k = L.zb[z];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        L.zt0[f][z] = 0u;
        L.ztn[f][z] = 0u;
        if (f >= NF || bcls(L.binfo[k], f) != kBTie) continue;
        const uint32_t key = k | ((uint32_t)f << 31);
        uint32_t lo = 0, hi = nt;  // a fold's ties in a bucket are a run of tord
        while (lo < hi) {
          const uint32_t mid = (lo + hi) >> 1;
          if (L.tbk[L.tord[mid]] < key) lo = mid + 1; else hi = mid;
        }
        uint32_t e = lo;
        while (e < nt && L.tbk[L.tord[e]] == key) ++e;
        L.zt0[f][z] = (uint16_t)lo;
        L.ztn[f][z] = (uint16_t)(e - lo);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t bi = L.binfo[k0 + j];
    const bool zone = bcls(bi, 0) >= kBZone || bcls(bi, 1) >= kBZone;  // gathered or split at ties
#pragma unroll
    for (int f = 0; f < NF; ++f)
      if (!zone && bcls(bi, f) == kBCert) atomicAdd(&L.seg[f][bslot(bi)], (unsigned long long)Df(f)[k0 + j]);
  }

  // Sort each gathering zone by (key desc, id asc), ranking by counting
  // larger packed values; then replace each key by the element's term, so
  // the replays read terms.
  for (uint32_t z = wave; z < nz; z += kWaves) {
    const uint32_t bz = L.binfo[L.zb[z]];
    if (bcls(bz, 0) != kBZone && bcls(bz, 1) != kBZone) continue;
    const uint32_t base = L.zbase[z], n = L.zcur[z];
    const unsigned long long* pk = L.zpk + base;
    for (uint32_t i = lane; i < n; i += 64u) {
      const unsigned long long me = pk[i];
      uint32_t r = 0;
      uint32_t j = 0;
      for (; j + 4u <= n; j += 4u)
        r += (pk[j] > me ? 1u : 0u) + (pk[j + 1] > me ? 1u : 0u) + (pk[j + 2] > me ? 1u : 0u) + (pk[j + 3] > me ? 1u : 0u);
      for (; j < n; ++j) r += pk[j] > me ? 1u : 0u;
      L.zperm[base + r] = (uint16_t)i;
    }
    for (uint32_t i = lane; i < n; i += 64u) {
      const unsigned long long v = L.zpk[base + i];
      const float t = term_of(glibc_expf_tab(key2f((uint32_t)(v >> 32)) - mx, L.exptab));
      L.zpk[base + i] = ((unsigned long long)__float_as_uint(t) << 32) | (uint32_t)v;
    }
  }
  lds_signal(&L.misc[kVSortDone]);

  // Waves 1 .. 15, each as soon as its share of the sort is done, sum each
  // tie bucket's ulp counts above each of its ties: they claim blocks of the
  // row (or of the list, when it covers every tie bucket) one at a time, so
  // the re-read overlaps the sort of the largest zones and wave 0's replay.
  // Wave 0 waits for them only when it reaches the first tie zone.
  if (wave != 0 && nt) {
    auto split = [&](float w, uint32_t i) __attribute__((always_inline)) {
      const float y = w - mx;
      const uint32_t k = vbucket(y);
      const uint32_t bi = L.binfo[k];
      if (bcls(bi, 0) != kBTie && bcls(bi, 1) != kBTie) return;
      const float t = term_of(glibc_expf_tab(y, L.exptab));
      if (thr > 0.0f && !(t >= thr)) return;
      const uint32_t z = bslot(bi);
      const uint32_t key = f2key(w);
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        if (bcls(bi, f) != kBTie) continue;
        bool tie, big;
        const uint32_t q = rne_units(t, bbin(bi, f), tie, big);
        if (tie || q == 0u) continue;
        const uint32_t t0 = L.zt0[f][z], tn = L.ztn[f][z];
        for (uint32_t v = 0; v < tn; ++v) {
          const uint32_t s = L.tord[t0 + v];
          if (before(key, i, L.tkey[s], L.tidx[s])) atomicAdd(&L.tab[s], q);
        }
      }
    };
    const bool from_list = tl_ok && L.misc[kVTieMax] <= tl_k;
    const uint32_t nb = from_list ? tl.blocks() : src.blocks();
    for (;;) {
      uint32_t blk = 0u;
      if (lane == 0) blk = atomicAdd(&L.misc[kVSplitNext], 1u);
      blk = readlane_u32(blk, 0);
      if (blk >= nb) break;
      // Only about 2% of the elements lie in tie buckets, but a wave would
      // run the tie work for an element position whenever one lane's
      // element there does. The lane's tie-bucket elements are found
      // first, then taken one at a time: the wave runs the tie work as many
      // times as its busiest lane has such elements.
      float w[16];
      uint32_t id[16], valid;
      if (from_list) tl.load_block(blk, w, id, valid);
      else src.load_block(blk, w, id, valid);
      uint32_t todo = 0u;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        if (!((valid >> e) & 1u)) continue;
        const uint32_t bi = L.binfo[vbucket(w[e] - mx)];
        todo |= (bcls(bi, 0) == kBTie || bcls(bi, 1) == kBTie) ? 1u << e : 0u;
      }
      while (todo != 0u) {
        const uint32_t e = (uint32_t)__builtin_ctz(todo);
        todo &= todo - 1u;
        float we = w[0];
        uint32_t ie = id[0];
#pragma unroll
        for (int q = 1; q < 16; ++q) {
          we = e == (uint32_t)q ? w[q] : we;
          ie = e == (uint32_t)q ? id[q] : ie;
        }
        split(we, ie);
      }
    }
    lds_signal(&L.misc[kVSplitDone]);
  }

  LLMHIP_MARK(NF == 1 ? 5 : 9);
  // Replays (wave 0), one fold after the other: certain segments as
  // integers, tie zones split at their ties, gathering zones 64 elements at a
  // time.
  if (wave == 0) {
    lds_wait(&L.misc[kVSortDone], kWaves, a);  // every zone sorted, every segment summed
    bool split_ready = nt == 0u;
    bool fail = false;
    uint32_t keep = keep_default;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (fail) break;
      const FoldSpec& sp = fs[f];
      const uint32_t kb = f == 0 ? kb0 : kb1;
      const uint32_t pos_end = f == 0 ? kNoPos : keep;
      float F = sp.F0;
      if (f == 1) F = u * res[0].F;  // generate.rs:411-412: r = u * total
      bool stopped = false;  // a stop, the end at keep, or past the last bucket
      bool at_keep = false;
      uint32_t stop_pos = kNoPos, stop_id = 0, stop_bk = 0;
      // Adds d ulps to F in binade E (add folds) or takes them away (the
      // walk); false when F would leave the binade.
      auto apply_units = [&](int E, uint64_t d) __attribute__((always_inline)) -> bool {
        const uint32_t fb = __float_as_uint(F), ef = (fb >> 23) & 255u;
        if (!(F > 0.0f) || ef == 0u || ef == 255u || (int)ef - 127 != E) return false;
        uint64_t M = (fb & 0x7fffffu) | 0x800000u;
        if (!sp.sub) {
          M += d;
          if (M >= (1ull << 24)) return false;
        } else {
          if (M < d + (1ull << 23) + 1ull) return false;
          M -= d;
        }
        F = from_units((uint32_t)M, E);
        return true;
      };
      // One element in f32, the reference's way; true when the fold stops.
      auto step = [&](float tv) __attribute__((always_inline)) -> bool {
        if (sp.sub) {
          if (F < tv) return true;
          F = F - tv;
          return false;
        }
        F = F + tv;
        return F >= sp.stop_ge;
      };
      for (uint32_t zc = 0; zc <= nz && !fail && !stopped; zc += 64u) {
        // Segment and zone data of zones zc .. zc + 63, one zone per lane, so
        // the walk through them reads registers.
        const uint32_t zl = zc + lane;
        uint32_t mSegE = (uint32_t)kNoE, mSegTub = 0u, mK = 0u, mBase = 0u, mN = 0u, mP0 = 0u, mBi = 0u;
        uint32_t mTub = 0u, mT0 = 0u, mTn = 0u, mD = 0u;
        uint64_t mSeg = 0ull;
        if (zl <= nz) {
          mSegE = (uint32_t)L.segE[f][zl];
          mSeg = L.seg[f][zl];
          if (sp.sub) mSegTub = L.segTub[zl];
        }
        if (zl < nz) {
          mK = L.zb[zl];
          mBase = L.zbase[zl];
          mN = L.zcur[zl];
          mP0 = L.zpos[zl];
          mBi = L.binfo[mK];
          if (sp.sub) mTub = __float_as_uint(term_of(glibc_expf_tab(-(float)mK / kVR, L.exptab)));  // largest term of the bucket
          mT0 = L.zt0[f][zl];
          mTn = L.ztn[f][zl];
          mD = Df(f)[mK];
        }
        for (uint32_t zi = 0; zi < 64u && zc + zi <= nz && !fail && !stopped; ++zi) {
          const uint32_t z = zc + zi;
          const int Es = (int)readlane_u32(mSegE, zi);
          if (Es != kNoE) {
            if (!apply_units(Es, readlane_u64(mSeg, zi))) fail = true;
            else if (!sp.sub && F >= sp.stop_ge) fail = true;
            else if (sp.sub && F < __uint_as_float(readlane_u32(mSegTub, zi))) fail = true;
          }
          if (z == nz || fail) break;
          const uint32_t k = readlane_u32(mK, zi);
          if (k >= kb) {  // past the fold's last bucket
            stopped = true;
            break;
          }
          const uint32_t bi = readlane_u32(mBi, zi);
          const uint32_t cf = bcls(bi, f);
          if (cf == kBSkip) continue;
          if (bcls(bi, 0) != kBZone && bcls(bi, 1) != kBZone) {
            // A tie zone: this fold's ties split it, or it is one certain bucket.
            const int E = bbin(bi, f);
            const uint32_t D = readlane_u32(mD, zi);
            uint32_t prev = 0;
            if (cf == kBTie) {
              if (!split_ready) {
                lds_wait(&L.misc[kVSplitDone], kWaves - 1u, a);
                split_ready = true;
              }
              const uint32_t t0 = readlane_u32(mT0, zi), tn = readlane_u32(mTn, zi);
              for (uint32_t v = 0; v < tn && !fail; ++v) {
                const uint32_t s = L.tord[t0 + v];
                const uint32_t ab = L.tab[s];
                if (!apply_units(E, ab - prev)) fail = true;
                prev = ab;
                const uint32_t q = L.tq[s];
                const uint32_t par = (__float_as_uint(F) ^ q) & 1u;  // parity of M - q or M + q
                if (!fail && !apply_units(E, (uint64_t)q + par)) fail = true;
              }
            }
            if (!fail && !apply_units(E, D - prev)) fail = true;
            if (!fail && !sp.sub && F >= sp.stop_ge) fail = true;
            if (!fail && sp.sub && F < __uint_as_float(readlane_u32(mTub, zi))) fail = true;
            continue;
          }
          const uint32_t base = readlane_u32(mBase, zi), n = readlane_u32(mN, zi), p0 = readlane_u32(mP0, zi);
          if (cf == kBCert && !(bi & (kBStep << f)) && p0 + n <= pos_end) {
            // Gathered for the other fold, certain for this one: one integer.
            if (!apply_units(bbin(bi, f), readlane_u32(mD, zi))) fail = true;
            else if (!sp.sub && F >= sp.stop_ge) fail = true;
            else if (sp.sub && F < __uint_as_float(readlane_u32(mTub, zi))) fail = true;
            if (!fail && p0 + n >= pos_end) at_keep = stopped = true;
            continue;
          }
          uint32_t r0 = 0;
          while (r0 < n && !stopped) {
            const uint32_t r = r0 + lane;
            float t = 0.0f;
            uint32_t id = 0u;
            if (r < n) {
              const unsigned long long v = L.zpk[base + L.zperm[base + r]];
              t = __uint_as_float((uint32_t)(v >> 32));
              id = ~(uint32_t)v;
            }
            const bool live = r < n;
            const bool past = live && p0 + r >= pos_end;
            const uint32_t fb = __float_as_uint(F), ef = (fb >> 23) & 255u;
            uint32_t done = 0u;  // lanes folded as integers before the one stepped in f32
            if (F > 0.0f && ef >= 1u && ef <= 254u) {
              const int E = (int)ef - 127;
              const uint32_t M = (fb & 0x7fffffu) | 0x800000u;
              bool tie = false, big = false;
              const uint32_t q = live && !past ? rne_units(t, E, tie, big) : 0u;
              const uint32_t incl = wave_incl_scan(q), excl = incl - q;
              bool ev;
              if (!sp.sub) {
                const uint64_t Mi = (uint64_t)M + incl;
                ev = tie || big || Mi >= (1ull << 24) || from_units((uint32_t)Mi, E) >= sp.stop_ge;
              } else {
                const bool ub = (uint64_t)excl + (1ull << 23) + 1ull > M;
                const bool ui = (uint64_t)incl + (1ull << 23) + 1ull > M;
                ev = tie || big || ub || ui || from_units(M - excl, E) < t;
              }
              ev = live && (ev || past);
              const uint64_t m = __ballot(ev);
              const uint32_t ev_lane = m ? (uint32_t)__ffsll((unsigned long long)m) - 1u : 64u;
              done = min(ev_lane, n - r0);
              if (done) {
                const uint32_t sum = readlane_u32(incl, done - 1u);
                const uint64_t M2 = sp.sub ? (uint64_t)M - sum : (uint64_t)M + sum;
                F = from_units((uint32_t)M2, E);
              }
            }
            if (r0 + done >= n) {
              r0 = n;
              break;
            }
            if (done == 64u) {  // no event in these 64
              r0 += 64u;
              continue;
            }
            // The event element (or the first one when F is not a normal number).
            const uint32_t le = done;
            const uint32_t pos = p0 + r0 + le;
            if (pos >= pos_end) {
              at_keep = stopped = true;  // the rest of the fold is outside it
              break;
            }
            if (step(readlane_f32(t, le))) {
              stop_pos = pos;
              stop_id = readlane_u32(id, le);
              stop_bk = k;
              stopped = true;
              break;
            }
            r0 += le + 1u;
          }
          // The walk ends with the zone that holds the cut (the last kept
          // element), whatever certain buckets follow it.
          if (!stopped && p0 + n >= pos_end) at_keep = stopped = true;
        }
      }
      // Past the end without a stop, although a bucket was certain to lie
      // past the stop: the approximation was wrong.
      if (!fail && stop_pos == kNoPos && !at_keep && kb < kVB) fail = true;
      res[f].F = F;
      res[f].stop_pos = stop_pos;
      res[f].stop_id = stop_id;
      res[f].stop_bk = stop_bk;
      if (f == 0) keep = stop_pos != kNoPos ? stop_pos + 1u : keep_count ? max(1u, L.misc[kVCount]) : keep_default;
    }
    if (lane == 0) {
      L.misc[kVFail] = fail ? 1u : 0u;
      L.misc[kVKeep] = keep;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        L.misc[kVRes + 4 * f + 0] = __float_as_uint(res[f].F);
        L.misc[kVRes + 4 * f + 1] = res[f].stop_pos;
        L.misc[kVRes + 4 * f + 2] = res[f].stop_id;
        L.misc[kVRes + 4 * f + 3] = res[f].stop_bk;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    res[f].F = __uint_as_float(L.misc[kVRes + 4 * f + 0]);
    res[f].stop_pos = L.misc[kVRes + 4 * f + 1];
    res[f].stop_id = L.misc[kVRes + 4 * f + 2];
    res[f].stop_bk = L.misc[kVRes + 4 * f + 3];
  }
  keep_out = L.misc[kVKeep];
  const bool ok = L.misc[kVFail] == 0u;
  __syncthreads();
  LLMHIP_MARK(NF == 1 ? 6 : 10);
  return ok;
}

// The three folds and the draw, given the row's source. Returns false
// (uniformly) when the row must go to general_row.
// raw: the same row before the division by T, and div_T that T (> 0,
// finite, normal) when the max pass may read it instead (else 0): w -> w / T
// rounded is monotone, so the largest quotient is the largest value's, and
// one division replaces one per element.
template <class Src, class RawSrc>
__device__ __forceinline__ bool vocab_folds(const SampleArgs& a, uint32_t b, uint32_t len_b, const llmhip_params& P, VocabLds& L,
                            const Src& src, const RawSrc& raw, float div_T) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t V = a.V;
  // Max; NaN and +inf rows take the sorting path.
  float mx = -INFINITY;
  uint32_t bad = 0u;
  auto max_of = [&](float w, uint32_t) __attribute__((always_inline)) {
    if (w != w || w == INFINITY) bad = 1u;
    mx = fmaxf(mx, w);
  };
  if (div_T > 0.0f) {
    raw.for_each(max_of);
  } else {
    src.for_each(max_of);
  }
#pragma unroll
  for (uint32_t off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (__ballot(bad != 0u) && lane == 0) L.misc[kVFail] = 1u;
  if (lane == 0) L.redf[wave] = mx;
  for (uint32_t k = tid; k < kVB; k += kBlock) {
    L.cnt[k] = 0u;
    L.asum[k] = 0.0f;
  }
  __syncthreads();
  mx = L.redf[0];
  for (uint32_t w = 1; w < kWaves; ++w) mx = fmaxf(mx, L.redf[w]);
  if (div_T > 0.0f) mx = mx / div_T;  // generate.rs:357-359 for the largest value
  if (L.misc[kVFail] || mx == -INFINITY || mx == INFINITY) return false;
  LLMHIP_MARK(1);

  // Bucket counts and approximate masses. The masses add up as integers
  // (x in units of 2^-40): LDS integer atomics are much faster than float ones.
  static_assert(sizeof(L.zpk) >= kVB * sizeof(unsigned long long), "amass");
  unsigned long long* amass = L.zpk;
  for (uint32_t k = tid; k < kVB; k += kBlock) amass[k] = 0ull;
  // With min-p on, elements of the buckets that can reach p >= min_p * p_0
  // (x >= ~min_p, so y >= ~ln(min_p); two buckets of slack) are listed. The
  // softmax sum's tie split reads the list too when every tie lies there.
  const uint32_t list_cap = (uint32_t)min((uint64_t)a.scratch_row_words / 2u, (uint64_t)kVListCap);
  const uint32_t kc = P.min_p > 0.0f && P.min_p <= 1.0f ? (uint32_t)fminf(-logf(P.min_p) * kVR + 2.0f, (float)(kVB - 1u)) : 0u;
  uint2* list = reinterpret_cast<uint2*>(a.scratch + (size_t)b * a.scratch_row_words);
  __syncthreads();
  src.for_each([&](float w, uint32_t i) __attribute__((always_inline)) {
    const float y = w - mx;
    const uint32_t k = vbucket(y);
    atomicAdd(&L.cnt[k], 1u);
    if (k <= kc && kc) {
      const uint32_t s = atomicAdd(&L.misc[kVCand], 1u);
      if (s < list_cap) list[s] = make_uint2(f2key(w), i);
    }
    const uint32_t xb = __float_as_uint(__expf(y));
    const int sh = (int)((xb >> 23) & 255u) - 127 + 17;  // x * 2^40 = m * 2^(e + 17)
    const unsigned long long m = (xb & 0x7fffffu) | 0x800000u;
    const unsigned long long fx = sh >= 0 ? (m << sh) : (sh > -24 ? (m >> -sh) : 0ull);
    if (fx) atomicAdd(&amass[k], fx);
  });
  __syncthreads();
  for (uint32_t k = tid; k < kVB; k += kBlock) L.asum[k] = (float)((double)amass[k] * 0x1p-40);
  __syncthreads();
  LLMHIP_MARK(2);

  // generate.rs:372-377: the softmax sum. The max element has x = 1, so S >= 1.
  const uint32_t ncand = L.misc[kVCand];
  const bool listed = kc && ncand <= list_cap;  // the list holds every element of buckets 0 .. kc
  const ListSrc lsrc{list, listed ? ncand : 0u};
  FoldSpec fs[1] = {{0.0f, 0.0f, 0.0f, INFINITY, false}};
  FoldRes r[1];
  uint32_t keep;
  if (!run_folds<1>(fs, mx, 0.0f, V, false, L, src, lsrc, listed, kc, r, keep, a)) return false;
  const float S = r[0].F;
  if (!(S > 0.0f) || !isfinite(S)) return false;

  // generate.rs:378-409: p = x / S; min-p by value (p is monotone along the
  // order); the top-p cumulative, whose value at the cut is the total. Then
  // generate.rs:411-419: r = u * total, and the walk.
  const float p0 = 1.0f / S;
  const float thr = P.min_p > 0.0f ? P.min_p * p0 : 0.0f;
  auto cut_and_walk = [&](const auto& from) __attribute__((always_inline)) -> bool {
    uint64_t st = a.rng_state[b];
    const float u = next_f32(st);
    FoldSpec fw[2] = {{0.0f, S, thr, P.top_p < 1.0f ? P.top_p : INFINITY, false},
                      {0.0f, S, thr, INFINITY, true}};
    FoldRes rw[2];
    uint32_t keep;
    if (!run_folds<2>(fw, mx, u, V, P.min_p > 0.0f, L, from, lsrc, listed, kc, rw, keep, a)) return false;
    // The walk's stop, else order[keep - 1] (the cut); without either the
    // row is handed over.
    const bool walk_stop = rw[1].stop_pos != kNoPos, cut = rw[0].stop_pos != kNoPos;
    const uint32_t id_walk = rw[1].stop_id, id_cut = rw[0].stop_id;
    if (!walk_stop && !cut) return false;
    const uint32_t pick = walk_stop ? id_walk : id_cut;
    if (tid == 0) {
      store_result(a, b, pick, len_b);
      a.rng_state[b] = st;
      if (a.out_kept) a.out_kept[b] = keep;
    }
    if (a.out_probs) {
      // generate.rs:378-380 and 384-409: p_i = e_i / S over the kept prefix
      // of the order, scattered by id into the row the caller has zeroed.
      // The prefix ends at the top-p cut (the element at sorted position
      // keep - 1, whose id the cumulative's replay found). Without a cut it
      // is min-p's: p never increases along the order, so it holds exactly
      // the elements with p >= thr. A prefix of one is order[0], which the
      // walk then picks.
      float* prow = a.out_probs + (size_t)b * V;
      if (keep == 1u) {
        if (tid == 0) prow[pick] = glibc_expf_tab(src.value_at(pick) - mx, L.exptab) / S;
      } else {
        const bool by_cut = cut;
        const uint64_t cut_ord = by_cut ? cand_order(f2key(src.value_at(id_cut)), id_cut) : 0ull;
        src.for_each([&](float w, uint32_t i) __attribute__((always_inline)) {
          const float pi = glibc_expf_tab(w - mx, L.exptab) / S;
          const bool kept = by_cut ? cand_order(f2key(w), i) >= cut_ord : pi >= thr;
          if (kept && pi != 0.0f) prow[i] = pi;
        });
      }
    }
    return true;
  };
  // The list holds every element the two folds can include when the first
  // bucket past it lies wholly below the min-p threshold.
  if (listed && kc + 1u < kVB && glibc_expf_tab(-(float)(kc + 1u) / kVR, L.exptab) / S < thr) {
    return cut_and_walk(lsrc);
  }
  return cut_and_walk(src);
}

// Returns false (uniformly) when the row must go to general_row. PLAIN: the
// call has no allowed mask, no ring and no row with a repetition penalty
// and a history; that variant is compiled without the mask, penalty and
// decode-step code (fewer values live through the passes).
// An element's value in parts (StreamSrc): the allowed mask
// (generate.rs:333-341), the penalized value of a history id (the mask, then
// one penalty step per occurrence, generate.rs:343-352, computed once per id
// into the LDS hash), and the division by T (generate.rs:357-359).
struct VocabVals {
  const uint8_t* allowed;
  const uint32_t* allowed_bits;
  uint32_t allowed_len, eos;
  bool use_pen;
  const VocabLds* L;
  bool div;
  float T;
  __device__ __forceinline__ float pre(uint32_t i, float v) const {
    if (allowed) {
      if (i < allowed_len && i != eos && allowed[i] == 0) v = -INFINITY;
    }
    if (allowed_bits) {
      if (i < allowed_len && i != eos && ((allowed_bits[i >> 5] >> (i & 31u)) & 1u) == 0u) v = -INFINITY;
    }
    return v;
  }
  __device__ __forceinline__ bool pen() const { return use_pen; }
  __device__ __forceinline__ bool hit(uint32_t i) const { return (L->hbits[(i >> 5) & (kVBits - 1u)] >> (i & 31u)) & 1u; }
  // Filter bits of ids i .. i + 3 (i a multiple of 4: one word holds them).
  __device__ __forceinline__ uint32_t hit4(uint32_t i) const { return (L->hbits[(i >> 5) & (kVBits - 1u)] >> (i & 31u)) & 15u; }
  // The filter holds ids modulo 2^17, so a hit may be no history id: v stays.
  __device__ __forceinline__ float hist(uint32_t i, float v) const {
    uint32_t h = (i * 2654435761u) >> 21;
    for (uint32_t probe = 0; probe < kVHash; ++probe) {
      const uint32_t k = L->hkey[h];
      if (k == i) return L->hval[h];
      if (k == kHashEmpty) break;
      h = (h + 1u) & (kVHash - 1u);
    }
    return v;
  }
  __device__ __forceinline__ float post(float v) const {
    if (div) {
      // The empty asm keeps the division inside the (row-uniform) branch:
      // left alone, the compiler computes it for every element and selects,
      // which costs rows with T == 1 a division each.
      float t = T;
      asm volatile("" : "+v"(t));
      v = v / t;
    }
    return v;
  }
};

template <bool PLAIN>
__device__ __forceinline__ bool vocab_row(const SampleArgs& a, uint32_t b, VocabLds& L, bool vec4) {
  const uint32_t tid = threadIdx.x;
  LLMHIP_MARK(0);
  const llmhip_params P = load_params(a, b);
  const uint32_t V = a.V;
  const float* row = a.logits + (size_t)b * a.ld;
  if (tid < 32) L.exptab[tid] = exp2f_tab_lane(tid);
  if (tid < kVMisc) L.misc[tid] = 0u;

  uint32_t h0 = 0, h1 = 0;
  if (!PLAIN && a.ring_cap) {
    h0 = a.ring_len[b];
    h1 = ring_avail(a, b, h0);
    if (a.done && a.done[b]) {
      if (tid == 0) {
        a.out_ids[b] = a.eos_id;
        if (a.out_kept) a.out_kept[b] = 0u;
      }
      return true;
    }
  } else if (!PLAIN && a.hist && a.hist_offsets) {
    h0 = a.hist_offsets[b];
    h1 = a.hist_offsets[b + 1];
  }
  const uint32_t len_b = h0;
  const HistRow hr = hist_row(a, b, h0, h1);
  // The count table is kept current for the next step; this path counts the
  // window itself.
  if (!PLAIN && a.ring_cap && a.counts) counts_advance_all(a, b, len_b, hr.H);
  const float rp = P.repetition_penalty, T = P.temperature;
  const bool use_pen = !PLAIN && rp != 1.0f && hr.H > 0;
  __syncthreads();

  // Repetition counts in an LDS hash (open addressing, probes bounded by the
  // table size), then each history id's penalized value (generate.rs:333-352:
  // the mask first, then one penalty step per occurrence).
  if (use_pen) {
    for (uint32_t s = tid; s < kVHash; s += kBlock) {
      L.hkey[s] = kHashEmpty;
      L.D[s] = 0u;
    }
    for (uint32_t s = tid; s < kVBits; s += kBlock) L.hbits[s] = 0u;
    __syncthreads();
    for (uint32_t j = tid; j < hr.H; j += kBlock) {
      const uint32_t id = hr.at(j);
      if (id >= V) continue;
      atomicOr(&L.hbits[(id >> 5) & (kVBits - 1u)], 1u << (id & 31u));
      uint32_t h = (id * 2654435761u) >> 21;
      for (uint32_t probe = 0; probe < kVHash; ++probe) {
        const uint32_t old = atomicCAS(&L.hkey[h], kHashEmpty, id);
        if (old == id || old == kHashEmpty) {
          if (old == kHashEmpty && atomicAdd(&L.misc[kVDistinct], 1u) >= kVMaxDistinct) L.misc[kVFail] = 1u;
          atomicAdd(&L.D[h], 1u);
          break;
        }
        h = (h + 1u) & (kVHash - 1u);
      }
    }
    __syncthreads();
    if (L.misc[kVFail]) return false;
    for (uint32_t s = tid; s < kVHash; s += kBlock) {
      const uint32_t id = L.hkey[s];
      if (id != kHashEmpty) {
        float v = row[id];
        if (masked_out(a, id)) v = -INFINITY;
        L.hval[s] = apply_penalty(v, L.D[s], rp);
      }
    }
    __syncthreads();
  }
  // Each test on a row-wide condition is a branch of its own, so rows with
  // no mask, no penalty or T == 1 pay nothing per element for it.
  const bool div_t = T != 1.0f;
  const VocabVals vv{PLAIN ? nullptr : a.allowed, PLAIN ? nullptr : a.allowed_bits, a.allowed_len, a.eos_id,
                     use_pen, &L, div_t, T};
  VocabVals vr = vv;
  vr.div = false;
  const StreamSrc<VocabVals> src{row, V, vec4, vv};
  const StreamSrc<VocabVals> raw{row, V, vec4, vr};
  const bool defer = div_t && T >= 0x1p-126f && T < INFINITY;
  return vocab_folds(a, b, len_b, P, L, src, raw, defer ? T : 0.0f);
}

}  // namespace llmhip
