// gfx950 kernels of the decode-time sampler.
//
// One 1024-thread workgroup (16 wave64s) samples one row, so a batch of B
// rows is B workgroups and B=256 fills the 256 CUs of an MI355X once. Two
// kernels share the row semantics of crates/llm-core/src/generate.rs:325-420:
//
//  * sample_fast_kernel (V <= 32768, 0 < top_k <= 1024, and greedy rows):
//    the row stays in registers. Each thread issues its 128-bit loads
//    up front (NCH dwordx4 per lane, each wave reading 1 KiB contiguous),
//    counts the history ids it prefetched before those loads into a u16
//    multiplicity table in LDS while the logits are in flight, then applies
//    mask -> penalty (m times in sequence by the lane that owns the logit, no
//    float atomics) -> temperature, and maps every value to an
//    order-preserving u32 key. An exact 4-pass LDS radix select finds the
//    K-th largest of the 1024 per-thread maxima; at least K elements lie at
//    or above it and at most K threads hold any, so the surviving candidate
//    set is tiny (about K for i.i.d. rows). Candidates are ranked by
//    (key desc, id asc) with a split all-pairs count and scattered into
//    sorted order; one wave then replays the reference's folds.
//
//  * sample_general_kernel (everything else: top_k == 0, top_k >= V, large
//    V, and rows the fast kernel cannot bound): a stable LSD radix sort of
//    (key, id) pairs in per-row HBM scratch gives exactly the reference's
//    `order`, followed by the same sequential tail.
#include "draw_tail.h"
#include "sampler_common.h"
#include "wave_ops.h"

namespace llmhip {

// LDS needed by the general path (about 19 KB).
struct GenLds {
  uint32_t bins[256];
  uint32_t off[256];
  uint32_t wc[kWaves * 256];
  float redv[kWaves];
  uint32_t redi[kWaves];
};

__device__ __forceinline__ llmhip_params load_params(const SampleArgs& a, uint32_t b) {
  return a.params ? a.params[(size_t)b * a.params_stride] : a.shared;
}

__device__ __forceinline__ float apply_penalty(float v, uint32_t m, float rp) {
  // generate.rs:343-352, once per occurrence, in sequence.
  for (; m; --m) v = v > 0.0f ? v / rp : v * rp;
  return v;
}

__device__ __forceinline__ bool masked_out(const SampleArgs& a, uint32_t id) {
  // generate.rs:333-341
  return a.allowed && id < a.allowed_len && id != a.eos_id && a.allowed[id] == 0;
}

// Block-wide argmax of (bv, bi) pairs; every thread must call. Returns the
// winner in all threads of wave 0 (UINT32_MAX when no thread had a value).
__device__ __forceinline__ uint32_t block_argmax(float bv, uint32_t bi, float* redv,
                                                 uint32_t* redi) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  wave_argmax(bv, bi);
  if (lane == 0) {
    redv[wave] = bv;
    redi[wave] = bi;
  }
  __syncthreads();
  float v = lane < kWaves ? redv[lane] : -INFINITY;
  uint32_t i = lane < kWaves ? redi[lane] : 0xffffffffu;
  wave_argmax(v, i);
  return i;
}

// ---------------------------------------------------------------------------
// General path: one row, 1024 threads, scratch in HBM.
// Scratch per row (Vp = V rounded up to 1024): keysA | idsA | keysB | idsB | cnt
// ---------------------------------------------------------------------------
__device__ void general_row(const SampleArgs& a, uint32_t b, const llmhip_params& P, GenLds& L) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t V = a.V;
  const uint32_t Vp = (V + kBlock - 1) / kBlock * kBlock;
  uint32_t* keysA = a.scratch + (size_t)b * a.scratch_row_words;
  uint32_t* idsA = keysA + Vp;
  uint32_t* keysB = idsA + Vp;
  uint32_t* idsB = keysB + Vp;
  uint32_t* cnt = idsB + Vp;
  const float* row = a.logits + (size_t)b * a.ld;

  bool use_pen = P.repetition_penalty != 1.0f && a.hist && a.hist_offsets;
  uint32_t h0 = 0, h1 = 0;
  if (use_pen) {
    h0 = a.hist_offsets[b];
    h1 = a.hist_offsets[b + 1];
    use_pen = h1 > h0;
  }
  if (use_pen) {
    // Integer multiplicities in L2 (device-scope atomics): order-independent.
    for (uint32_t i = tid; i < V; i += kBlock)
      __hip_atomic_store(&cnt[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    for (uint32_t j = h0 + tid; j < h1; j += kBlock) {
      const uint32_t id = a.hist[j];
      if (id < V) atomicAdd(&cnt[id], 1u);
    }
    __syncthreads();
  }

  const bool greedy = P.temperature <= 0.0f;
  const float T = P.temperature, rp = P.repetition_penalty;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  for (uint32_t i = tid; i < V; i += kBlock) {
    float v = row[i];
    if (masked_out(a, i)) v = -INFINITY;
    if (use_pen) v = apply_penalty(v, __hip_atomic_load(&cnt[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), rp);
    if (greedy) {
      if (v > bv) {
        bv = v;
        bi = i;
      }
    } else {
      keysA[i] = f2key(v / T);
      idsA[i] = i;
    }
  }
  if (greedy) {
    const uint32_t w = block_argmax(bv, bi, L.redv, L.redi);
    if (tid == 0) {
      a.out_ids[b] = w == 0xffffffffu ? 0u : w;
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }
  __syncthreads();

  // Stable LSD radix sort, 4 x 8-bit digits, descending: ties keep
  // ascending id, which is the reference's order (generate.rs:364-367).
  for (uint32_t pass = 0; pass < 4; ++pass) {
    const uint32_t shift = 8u * pass;
    const uint32_t* sK = (pass & 1) ? keysB : keysA;
    const uint32_t* sI = (pass & 1) ? idsB : idsA;
    uint32_t* dK = (pass & 1) ? keysA : keysB;
    uint32_t* dI = (pass & 1) ? idsA : idsB;
    if (tid < 256) L.bins[tid] = 0u;
    for (uint32_t i = tid; i < kWaves * 256; i += kBlock) L.wc[i] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < V; i += kBlock) atomicAdd(&L.bins[(sK[i] >> shift) & 255u], 1u);
    __syncthreads();
    if (wave == 0) {
      const uint32_t d0 = 255u - 4u * lane;
      const uint32_t c0 = L.bins[d0], c1 = L.bins[d0 - 1], c2 = L.bins[d0 - 2], c3 = L.bins[d0 - 3];
      const uint32_t tot = c0 + c1 + c2 + c3;
      const uint32_t ex = wave_incl_scan(tot) - tot;
      L.off[d0] = ex;
      L.off[d0 - 1] = ex + c0;
      L.off[d0 - 2] = ex + c0 + c1;
      L.off[d0 - 3] = ex + c0 + c1 + c2;
    }
    __syncthreads();
    for (uint32_t base = 0; base < V; base += kBlock) {
      const uint32_t i = base + tid;
      const bool valid = i < V;
      const uint32_t k = valid ? sK[i] : 0u;
      const uint32_t id = valid ? sI[i] : 0u;
      const uint32_t d = (k >> shift) & 255u;
      uint64_t m = __ballot(valid);
#pragma unroll
      for (uint32_t bit = 0; bit < 8; ++bit) {
        const bool s = (d >> bit) & 1u;
        const uint64_t bb = __ballot(s);
        m &= s ? bb : ~bb;
      }
      const uint32_t rank = (uint32_t)__popcll(m & lanemask_lt());
      if (valid && rank == 0) L.wc[wave * 256 + d] = (uint32_t)__popcll(m);
      __syncthreads();
      if (valid) {
        uint32_t pos = L.off[d] + rank;
        for (uint32_t w = 0; w < wave; ++w) pos += L.wc[w * 256 + d];
        dK[pos] = k;
        dI[pos] = id;
      }
      __syncthreads();
      if (tid < 256) {
        uint32_t s = 0;
        for (uint32_t w = 0; w < kWaves; ++w) {
          s += L.wc[w * 256 + tid];
          L.wc[w * 256 + tid] = 0u;
        }
        L.off[tid] += s;
      }
      __syncthreads();
    }
  }
  // Four passes end in A.
  const uint32_t n = (P.top_k > 0 && P.top_k < V) ? P.top_k : V;
  if (wave == 0) {
    draw_tail(a, b, P, n, [&](uint32_t i) { return keysA[i]; }, [&](uint32_t i) { return idsA[i]; });
  }
}

__global__ __launch_bounds__(kBlock) void sample_general_kernel(SampleArgs a) {
  __shared__ GenLds L;
  const uint32_t b = blockIdx.x;
  if (b >= a.B) return;
  const llmhip_params P = load_params(a, b);
  if (!(row_class(P, a.V) & a.row_class_mask)) return;
  general_row(a, b, P, L);
}

// ---------------------------------------------------------------------------
// Fast path: V <= 32768, row in registers.
// ---------------------------------------------------------------------------

// Workgroup barrier that orders LDS only: outstanding global loads stay in
// flight across it (a full __syncthreads would wait for every logits load).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

constexpr uint32_t kMaxPen = 4096;    // distinct penalized ids per row (register path)
constexpr uint32_t kFastCand = 2048;  // candidate buffer (register path)
constexpr uint32_t kPenPerThread = kMaxPen / kBlock;

// Element e of thread t holds position ((e/4)*1024 + t)*4 + e%4: each wave
// reads 1 KiB contiguous per dwordx4 load. Position p lives in thread
// (p/4) % 1024, slot ((p/4096)*4 + p%4).
__device__ __forceinline__ uint32_t slot_pos(uint32_t e, uint32_t tid) {
  return ((e >> 2) * kBlock + tid) * 4u + (e & 3u);
}
__device__ __forceinline__ uint32_t pos_owner(uint32_t p) { return (p >> 2) & (kBlock - 1); }
__device__ __forceinline__ uint32_t pos_slot(uint32_t p) { return ((p >> 12) << 2) | (p & 3u); }

template <int NCH, bool ALIGNED>
__global__ __launch_bounds__(kBlock) void sample_fast_kernel(SampleArgs a) {
  // u16 history multiplicity per id (2 per word); reused as the
  // general-path LDS when a row falls back.
  __shared__ uint32_t s_cnt[kMaxFastV / 2];
  __shared__ uint32_t s_pm[kBlock];      // per-thread mask of slots whose logit is penalized
  __shared__ uint32_t s_plist[kMaxPen];  // distinct penalized ids
  __shared__ uint32_t s_hist[4 * 256];
  __shared__ uint32_t s_ckey[kFastCand];
  __shared__ uint32_t s_cid[kFastCand];
  __shared__ uint32_t s_rank[kFastCand];
  __shared__ uint32_t s_skey[kMaxFastK];
  __shared__ uint32_t s_sid[kMaxFastK];
  __shared__ float s_redv[kWaves];
  __shared__ uint32_t s_redi[kWaves];
  __shared__ uint32_t s_misc[8];
  static_assert(sizeof(GenLds) <= sizeof(s_cnt), "general-path LDS must fit the count table");
  static_assert(NCH * 4 <= 32, "slot mask is 32 bits");

  const uint32_t b = blockIdx.x;
  if (b >= a.B) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const llmhip_params P = load_params(a, b);
  const uint32_t V = a.V;
  const uint32_t cls = row_class(P, V);
  if (!(cls & a.row_class_mask)) return;
  const float T = P.temperature, rp = P.repetition_penalty;

  bool use_pen = P.repetition_penalty != 1.0f && a.hist && a.hist_offsets;
  uint32_t h0 = 0, h1 = 0;
  if (use_pen) {
    h0 = a.hist_offsets[b];
    h1 = a.hist_offsets[b + 1];
    use_pen = h1 > h0;
    if (use_pen && h1 - h0 >= 65536u) {
      // A u16 count could overflow: take the general path.
      general_row(a, b, P, *reinterpret_cast<GenLds*>(s_cnt));
      return;
    }
  }
  // History ids are loaded before the logits so the counting below only
  // waits for them, not for the row.
  uint32_t hid0 = 0xffffffffu, hid1 = 0xffffffffu;
  if (use_pen) {
    if (h0 + tid < h1) hid0 = a.hist[h0 + tid];
    if (h0 + kBlock + tid < h1) hid1 = a.hist[h0 + kBlock + tid];
  }

  // All row loads in flight at once: NCH dwordx4 per lane.
  const float* row = a.logits + (size_t)b * a.ld;
  float x[NCH * 4];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const uint32_t base = ((uint32_t)c * kBlock + tid) * 4u;
    if (ALIGNED && base + 4u <= V) {
      const float4 q = *reinterpret_cast<const float4*>(row + base);
      x[4 * c + 0] = q.x;
      x[4 * c + 1] = q.y;
      x[4 * c + 2] = q.z;
      x[4 * c + 3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * c + j] = (base + j < V) ? row[base + j] : 0.0f;
    }
  }

  if (use_pen) {
    for (uint32_t i = tid; i < (V + 1) / 2; i += kBlock) s_cnt[i] = 0u;
    s_pm[tid] = 0u;
  }
  s_hist[tid] = 0u;  // 4 x 256 bins == kBlock
  if (tid < 8) s_misc[tid] = 0u;
  lds_barrier();

  // History multiplicities (integer LDS atomics: the counts do not depend
  // on the order). The first occurrence of an id enlists it for one
  // processor lane and marks its slot in the owner's mask.
  uint32_t D = 0;
  if (use_pen) {
    auto add_hist = [&](uint32_t id) {
      if (id < V) {
        const uint32_t sh = (id & 1u) << 4;
        const uint32_t old = atomicAdd(&s_cnt[id >> 1], 1u << sh);
        if (((old >> sh) & 0xffffu) == 0u) {
          const uint32_t q = atomicAdd(&s_misc[3], 1u);
          if (q < kMaxPen) s_plist[q] = id;
          atomicOr(&s_pm[pos_owner(id)], 1u << pos_slot(id));
        }
      }
    };
    add_hist(hid0);
    add_hist(hid1);
    for (uint32_t j = h0 + 2u * kBlock + tid; j < h1; j += kBlock) add_hist(a.hist[j]);
    lds_barrier();
    D = s_misc[3];
    if (D > kMaxPen) {
      __syncthreads();
      general_row(a, b, P, *reinterpret_cast<GenLds*>(s_cnt));
      return;
    }
  }

  // Processor lanes: each distinct penalized id is gathered once (its line
  // is being streamed by the row loads, so this merges in L2) and given
  // mask -> penalty (m times in sequence: no float atomics) here.
  float gv[kPenPerThread];
  uint32_t gp[kPenPerThread], gm[kPenPerThread];
#pragma unroll
  for (uint32_t r = 0; r < kPenPerThread; ++r) {
    const uint32_t q = tid + r * kBlock;
    gp[r] = 0xffffffffu;
    gm[r] = 0u;
    gv[r] = 0.0f;
    if (q < D) {
      const uint32_t p = s_plist[q];
      gp[r] = p;
      gm[r] = (s_cnt[p >> 1] >> ((p & 1u) << 4)) & 0xffffu;
      gv[r] = row[p];
    }
  }
  const uint32_t pm = use_pen ? s_pm[tid] : 0u;

  if (cls == kClassGreedy) {
    // ops/loss.rs:6-16 over the penalized, masked row (before temperature).
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) {
      const uint32_t pos = slot_pos(e, tid);
      float v = x[e];
      if (a.allowed && masked_out(a, pos)) v = -INFINITY;
      if (pos < V && !((pm >> e) & 1u) && v > bv) {
        bv = v;
        bi = pos;
      }
    }
#pragma unroll
    for (uint32_t r = 0; r < kPenPerThread; ++r) {
      if (gp[r] != 0xffffffffu) {
        float v = gv[r];
        if (masked_out(a, gp[r])) v = -INFINITY;
        v = apply_penalty(v, gm[r], rp);
        if (v > -INFINITY) argmax_combine(bv, bi, v, gp[r]);
      }
    }
    const uint32_t w = block_argmax(bv, bi, s_redv, s_redi);
    if (tid == 0) {
      a.out_ids[b] = w == 0xffffffffu ? 0u : w;
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }

  // Keys of the pre-temperature values v (mask applied; penalized logits
  // are represented by their processor lane instead). Dividing by T > 0
  // is monotone, so the top-k by v contains the top-k by v/T except for
  // values that the division merges into ties; those are caught below.
  uint32_t key[NCH * 4];
  uint32_t tmax = kKeyNone;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    const uint32_t pos = slot_pos(e, tid);
    float v = x[e];
    if (a.allowed && masked_out(a, pos)) v = -INFINITY;
    uint32_t k = f2key(v);
    if (pos >= V || ((pm >> e) & 1u)) k = kKeyNone;
    key[e] = k;
    tmax = k > tmax ? k : tmax;
  }
  uint32_t gk[kPenPerThread];
#pragma unroll
  for (uint32_t r = 0; r < kPenPerThread; ++r) {
    gk[r] = kKeyNone;
    if (gp[r] != 0xffffffffu) {
      float v = gv[r];
      if (masked_out(a, gp[r])) v = -INFINITY;
      gk[r] = f2key(apply_penalty(v, gm[r], rp));
      tmax = gk[r] > tmax ? gk[r] : tmax;
    }
  }

  // tau = exact K-th largest of the 1024 per-thread maxima (4 x 8-bit LDS
  // radix passes, bins scanned from the top by wave 0). At least K
  // elements have key >= tau and they live in at most K threads.
  const uint32_t K = P.top_k;  // 0 < K < V, K <= 1024 (row class)
  uint32_t prefix = 0u, kk = K;
#pragma unroll
  for (uint32_t pass = 0; pass < 4; ++pass) {
    const uint32_t shift = 24u - 8u * pass;
    const uint32_t hi_mask = pass == 0 ? 0u : (0xffffffffu << (shift + 8u));
    if ((tmax & hi_mask) == prefix) atomicAdd(&s_hist[pass * 256u + ((tmax >> shift) & 255u)], 1u);
    lds_barrier();
    if (wave == 0) {
      const uint32_t d0 = 255u - 4u * lane;
      const uint32_t* h = s_hist + pass * 256u;
      const uint32_t c0 = h[d0], c1 = h[d0 - 1], c2 = h[d0 - 2], c3 = h[d0 - 3];
      const uint32_t tot = c0 + c1 + c2 + c3;
      const uint32_t incl = wave_incl_scan(tot);
      uint32_t cum = incl - tot;
      uint32_t np = 0u, nk = 0u;
      const bool mine = cum < kk && kk <= incl;
      if (mine) {
        uint32_t d;
        if (cum + c0 >= kk) {
          d = d0;
        } else if (cum += c0, cum + c1 >= kk) {
          d = d0 - 1;
        } else if (cum += c1, cum + c2 >= kk) {
          d = d0 - 2;
        } else {
          cum += c2;
          d = d0 - 3;
        }
        np = prefix | (d << shift);
        nk = kk - cum;
      }
      const uint64_t who = __ballot(mine);
      const uint32_t src = who ? (uint32_t)__ffsll((unsigned long long)who) - 1u : 0u;
      np = readlane_u32(np, src);
      nk = readlane_u32(nk, src);
      if (pass < 3) {
        if (lane == 0) {
          s_misc[0] = np;
          s_misc[1] = nk;
        }
      } else {
        // Lowest v key whose v/T equals (tau)/T: the candidate threshold.
        // Lane l tests the value l+1 keys below tau; the run of ties from
        // the top is at most ceil(2T)+1 long, so one wave covers T < 31.
        uint32_t lo = np;
        if (np > kKeyNaN + 64u) {
          const uint32_t wt = f2key(key2f(np) / T);
          const bool tie = f2key(key2f(np - 1u - lane) / T) == wt;
          const uint64_t ties = __ballot(tie);
          const uint64_t run = ~ties;
          if (run == 0ull) {
            lo = kKeyNaN;  // more than 64 tied values: take everything
          } else {
            lo = np - (uint32_t)(__ffsll((unsigned long long)run) - 1);
          }
        } else {
          lo = kKeyNaN;
        }
        if (lane == 0) {
          s_misc[0] = np;
          s_misc[1] = lo;
        }
      }
    }
    lds_barrier();
    prefix = s_misc[0];
    kk = s_misc[1];
  }
  // After the last pass s_misc[1] holds the threshold.
  const uint32_t thr = kk > kKeyNaN ? kk : kKeyNaN;

  // Append candidates (key >= thr) with their post-temperature key: one
  // LDS atomic per wave, one division per candidate.
  uint32_t mine = 0u;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) mine += key[e] >= thr ? 1u : 0u;
#pragma unroll
  for (uint32_t r = 0; r < kPenPerThread; ++r) mine += gk[r] >= thr ? 1u : 0u;
  const uint32_t incl = wave_incl_scan(mine);
  const uint32_t wtot = readlane_u32(incl, 63);
  uint32_t wbase = 0u;
  if (lane == 0 && wtot) wbase = atomicAdd(&s_misc[2], wtot);
  wbase = readlane_u32(wbase, 0);
  uint32_t slot = wbase + incl - mine;
#pragma unroll
  for (int e = 0; e < NCH * 4; ++e) {
    if (key[e] >= thr) {
      if (slot < kFastCand) {
        s_ckey[slot] = f2key(key2f(key[e]) / T);
        s_cid[slot] = slot_pos(e, tid);
      }
      ++slot;
    }
  }
#pragma unroll
  for (uint32_t r = 0; r < kPenPerThread; ++r) {
    if (gk[r] >= thr) {
      if (slot < kFastCand) {
        s_ckey[slot] = f2key(key2f(gk[r]) / T);
        s_cid[slot] = gp[r];
      }
      ++slot;
    }
  }
  lds_barrier();
  const uint32_t n = s_misc[2];
  if (n > kFastCand) {
    // Heavy ties at the threshold: not bounded by the register path.
    __syncthreads();
    general_row(a, b, P, *reinterpret_cast<GenLds*>(s_cnt));
    return;
  }

  // Rank by (w key desc, id asc): rank(i) = #{j : cand j precedes cand i},
  // the j range split over all waves.
  for (uint32_t i = tid; i < n; i += kBlock) s_rank[i] = 0u;
  lds_barrier();
  if (n <= kBlock) {
    const uint32_t n64 = (n + 63u) & ~63u;
    const uint32_t groups = n64 ? kBlock / n64 : 1u;
    const uint32_t i = n64 ? tid % n64 : 0u, g = n64 ? tid / n64 : 0u;
    if (g < groups && i < n) {
      const uint32_t ki = s_ckey[i], ii = s_cid[i];
      const uint32_t j0 = n * g / groups, j1 = n * (g + 1) / groups;
      uint32_t r = 0u;
      for (uint32_t j = j0; j < j1; ++j) {
        const uint32_t kj = s_ckey[j], ij = s_cid[j];
        r += (kj > ki || (kj == ki && ij < ii)) ? 1u : 0u;
      }
      atomicAdd(&s_rank[i], r);
    }
  } else {
    for (uint32_t i = tid; i < n; i += kBlock) {
      const uint32_t ki = s_ckey[i], ii = s_cid[i];
      uint32_t r = 0u;
      for (uint32_t j = 0; j < n; ++j) {
        const uint32_t kj = s_ckey[j], ij = s_cid[j];
        r += (kj > ki || (kj == ki && ij < ii)) ? 1u : 0u;
      }
      s_rank[i] = r;
    }
  }
  lds_barrier();
  for (uint32_t i = tid; i < n; i += kBlock) {
    const uint32_t r = s_rank[i];
    if (r < K) {
      s_skey[r] = s_ckey[i];
      s_sid[r] = s_cid[i];
    }
  }
  lds_barrier();
  if (wave == 0) {
    draw_tail(a, b, P, K, [&](uint32_t i) { return s_skey[i]; }, [&](uint32_t i) { return s_sid[i]; });
  }
}

// ---------------------------------------------------------------------------
// Host-side launch.
// ---------------------------------------------------------------------------
template <int NCH>
static hipError_t launch_fast_nch(const SampleArgs& a, bool aligned, hipStream_t s) {
  if (aligned) {
    hipLaunchKernelGGL((sample_fast_kernel<NCH, true>), dim3(a.B), dim3(kBlock), 0, s, a);
  } else {
    hipLaunchKernelGGL((sample_fast_kernel<NCH, false>), dim3(a.B), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_fast(const SampleArgs& a, bool aligned, hipStream_t s) {
  if (a.V <= 4096) return launch_fast_nch<1>(a, aligned, s);
  if (a.V <= 8192) return launch_fast_nch<2>(a, aligned, s);
  if (a.V <= 16384) return launch_fast_nch<4>(a, aligned, s);
  return launch_fast_nch<8>(a, aligned, s);
}

hipError_t launch_general(const SampleArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(sample_general_kernel, dim3(a.B), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace llmhip
