// The general path of the gfx950 sampler: one row per 1024-thread
// workgroup with per-row scratch in HBM, for the rows the register path
// does not take (and the rows it hands over). Row semantics:
// crates/llm-core/src/generate.rs:325-420.
#pragma once
#include "draw_tail.h"
#include "fast_row.h"
#include "sampler_common.h"
#include "wave_ops.h"

namespace llmhip {

// ---------------------------------------------------------------------------
// Top-k selection for the general path (0 < K <= kSelCap, K < V): the K
// largest (key, id) pairs in the reference's order (key descending, ties by
// ascending id, generate.rs:364-367), from the keys of a row in scratch.
// ---------------------------------------------------------------------------

// Order key: larger means earlier in the sorted order.
__device__ __forceinline__ uint64_t sel_order(uint32_t key, uint32_t id) {
  return ((uint64_t)key << 32) | (uint32_t)~id;
}

// The K-th largest key t, by an MSB-first radix select (digits of 11, 11
// and 10 bits; bin counts from integer LDS atomics, so they do not depend on
// the order of the adds), and r: how many of the K largest keys equal t
// (1 <= r <= the count of t).
__device__ __forceinline__ void select_kth(const uint32_t* keys, uint32_t V, uint32_t K, GenLds& L, uint32_t& t,
                                           uint32_t& r) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  uint32_t* hist = L.wc;  // 2048 bins
  uint32_t prefix = 0u, pmask = 0u, need = K;
  for (uint32_t d = 0; d < 3u; ++d) {
    const uint32_t bits = d < 2u ? 11u : 10u, shift = d == 0u ? 21u : d == 1u ? 10u : 0u;
    const uint32_t nb = 1u << bits, per = nb / 64u;
    for (uint32_t i = tid; i < nb; i += kBlock) hist[i] = 0u;
    __syncthreads();
    for (uint32_t i0 = tid; i0 < V; i0 += 8u * kBlock) {
      uint32_t k[8];
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) k[u] = i0 + u * kBlock < V ? keys[i0 + u * kBlock] : 0u;
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u)
        if (i0 + u * kBlock < V && (k[u] & pmask) == prefix) atomicAdd(&hist[(k[u] >> shift) & (nb - 1u)], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      // Lane l holds bins top .. top - per + 1 (descending); the class holds
      // at least `need` keys, so some lane's inclusive count reaches it.
      const uint32_t top = nb - 1u - per * lane;
      uint32_t s = 0u;
      for (uint32_t j = 0; j < per; ++j) s += hist[top - j];
      const uint32_t inc = wave_incl_scan(s);
      const uint32_t l = (uint32_t)__ffsll((unsigned long long)__ballot(inc >= need)) - 1u;
      if (lane == l) {
        uint32_t c = inc - s, dg = top;
        for (uint32_t j = 0; j < per; ++j) {
          const uint32_t h = hist[top - j];
          if (c + h >= need) {
            dg = top - j;
            break;
          }
          c += h;
        }
        L.sv[0] = dg;
        L.sv[1] = c;
      }
    }
    __syncthreads();
    need -= L.sv[1];
    prefix |= L.sv[0] << shift;
    pmask |= (nb - 1u) << shift;
    __syncthreads();  // sv and the bins are rewritten by the next digit
  }
  t = prefix;
  r = need;
}

// L.sel[0, K) = the K largest order keys, sorted descending.
__device__ __forceinline__ void select_top(const uint32_t* keys, uint32_t V, uint32_t K, GenLds& L) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  uint32_t t, r;
  select_kth(keys, V, K, L, t, r);
  // Wave w walks the ids [w*R, (w+1)*R) in steps of 64 consecutive ids, 8
  // steps in flight: every load is coalesced, and each wave meets its ids
  // in ascending order. The keys above t (exactly K - r of them) go to
  // [0, K - r) in any order (the sort below orders them); the keys equal to
  // t are counted per wave.
  if (tid == 0) L.sv[2] = 0u;
  __syncthreads();
  const uint32_t R = ((V + kWaves - 1u) / kWaves + 63u) & ~63u;
  const uint32_t w0 = wave * R, w1 = min(V, w0 + R);
  uint32_t ties = 0u;  // this wave's keys equal to t
  for (uint32_t j0 = w0; j0 < w1; j0 += 8u * 64u) {
    uint32_t kb[8];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t i = j0 + u * 64u + lane;
      kb[u] = i < w1 ? keys[i] : 0u;
    }
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t i = j0 + u * 64u + lane, k = kb[u];
      const bool above = i < w1 && k > t;
      ties += (uint32_t)__popcll((unsigned long long)__ballot(i < w1 && k == t));
      const uint64_t m = __ballot(above);
      if (m) {
        uint32_t o = 0u;
        if (lane == 0) o = atomicAdd(&L.sv[2], (uint32_t)__popcll((unsigned long long)m));
        o = readlane_u32(o, 0) + lanes_below(m);
        if (above) L.sel[o] = sel_order(k, i);
      }
    }
  }
  if (lane == 0) L.redi[wave] = ties;
  __syncthreads();
  // The r lowest ids among the keys equal to t go to [K - r, K): the waves'
  // ranges are in id order, so a key's place among them is the ties of the
  // waves before its own, then of its wave's earlier steps and lanes.
  uint32_t rank = 0u;
  for (uint32_t w = 0; w < wave; ++w) rank += L.redi[w];
  if (ties != 0u && rank < r) {
    for (uint32_t j0 = w0; j0 < w1 && rank < r; j0 += 64u) {
      const uint32_t i = j0 + lane;
      const bool tie = i < w1 && keys[i] == t;
      const uint64_t m = __ballot(tie);
      if (tie) {
        const uint32_t q = rank + lanes_below(m);
        if (q < r) L.sel[K - r + q] = sel_order(t, i);
      }
      rank += (uint32_t)__popcll((unsigned long long)m);
    }
  }
  bitonic_sort_desc(L.sel, K);  // its first barrier completes the list
}

// select_top for keys taken before the division by T (keys[i] = f2key(v_i)):
// division is monotone, so every value of the top K after it (ties by id)
// lies at or above tlo, the lowest raw key whose quotient equals that of
// any raw key t0 at or below the K-th largest, and only those values are
// divided and sorted. When tlo is not bounded (a tie run longer than 64
// keys, or a t0 at -inf or NaN) or the candidates outnumber the list, every
// key is divided in place and select_top runs on them. Returns the sorted
// list: L.sel, or L.wc's words read as order keys when the listed values
// (at most 2048) were merge-sorted with L.sel as the first buffer.
__device__ __forceinline__ const uint64_t* select_top_raw(uint32_t* keys, uint32_t V, uint32_t K, float T,
                                                          GenLds& L) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  // t0: for K <= kSelCap / 2, the lower edge of the fine bin holding the
  // K-th largest group maximum (L.wc, counted by the keys pass), so at
  // least K values lie at or above it and t0 is at or below the K-th largest
  // raw key (about 1.1-1.3 K values are listed); for a larger K, whose group
  // bound would list more than the list holds, the K-th largest raw key
  // itself, by the radix select.
  uint32_t t0;
  if (K <= kSelCap / 2u) {
    coarse_from_fine(L.wc, L.bins);
    __syncthreads();
    t0 = hist_locate(L.bins, L.wc, K, lane).lo;  // the same in every wave
  } else {
    uint32_t r;
    select_kth(keys, V, K, L, t0, r);
  }
  const uint32_t tlo = t0 ? lower_past_ties(t0, T, lane) : 0u;
  uint32_t c = 0u;
  if (tid == 0) L.sv[2] = 0u;
  __syncthreads();  // every wave is past the histogram, which the fallback's select reuses
  if (tlo != 0u) {
    // Coalesced, as in select_top: wave w walks ids [w*R, (w+1)*R).
    const uint32_t R = ((V + kWaves - 1u) / kWaves + 63u) & ~63u;
    const uint32_t w0 = wave * R, w1 = min(V, w0 + R);
    for (uint32_t j0 = w0; j0 < w1; j0 += 8u * 64u) {
      uint32_t kb[8];
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        const uint32_t i = j0 + u * 64u + lane;
        kb[u] = i < w1 ? keys[i] : 0u;
      }
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        const uint32_t i = j0 + u * 64u + lane, k = kb[u];
        const bool cand = i < w1 && k >= tlo;
        const uint64_t m = __ballot(cand);
        if (m) {
          uint32_t o = 0u;
          if (lane == 0) o = atomicAdd(&L.sv[2], (uint32_t)__popcll((unsigned long long)m));
          o = readlane_u32(o, 0) + lanes_below(m);
          if (cand && o < kSelCap) L.sel[o] = sel_order(f2key(key2f(k) / T), i);
        }
      }
    }
    __syncthreads();
    c = L.sv[2];  // >= K: every value at or above t0 is a candidate
  }
  // The first K of the sorted list are the row's top K.
  if (tlo != 0u && c <= kSelCap) {
    static_assert(sizeof(L.wc) >= 2u * kBlock * sizeof(uint64_t), "the merge's second buffer");
    uint64_t* tmp = reinterpret_cast<uint64_t*>(L.wc);
    if (c <= kBlock) return sort_desc_lds<1>(L.sel, tmp, c);
    if (c <= 2u * kBlock) return sort_desc_lds<2>(L.sel, tmp, c);
    bitonic_sort_desc(L.sel, c);
    return L.sel;
  }
  for (uint32_t i = tid; i < V; i += kBlock) keys[i] = f2key(key2f(keys[i]) / T);
  __syncthreads();
  select_top(keys, V, K, L);
  return L.sel;
}

// ---------------------------------------------------------------------------
// General path: one row, 1024 threads, scratch in HBM.
// Scratch per row (Vp = V rounded up to 1024): keysA | cnt | idsA | keysB |
// idsB. Greedy rows and top-k rows that select in LDS touch only the first
// two (kScratchSelWords), so a call without whole-row sorts needs 2*Vp words
// per row; the sort needs all five (kScratchSortWords).
// ---------------------------------------------------------------------------
// counts_moved: the row's count table (decode-step mode with counts) was
// already moved to this step's window by the kernel that handed it over.
// SORT = false leaves out the whole-row sort, for the register path's
// hand-overs: those are greedy rows and top-k rows with K <= kMaxFastK,
// which select in LDS (K <= kSelCap), and the kernel is 20 KB of code
// smaller.
template <bool SORT = true>
__device__ __forceinline__ void general_row(const SampleArgs& a, uint32_t b, GenLds& L, bool counts_moved) {
  const llmhip_params P = load_params(a, b);
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t V = a.V;
  const uint32_t Vp = (V + kBlock - 1) / kBlock * kBlock;
  uint32_t* keysA = a.scratch + (size_t)b * a.scratch_row_words;
  uint32_t* cnt = keysA + Vp;
  uint32_t* idsA = cnt + Vp;
  uint32_t* keysB = idsA + Vp;
  uint32_t* idsB = keysB + Vp;
  const float* row = a.logits + (size_t)b * a.ld;
  if (tid < 32) L.exptab[tid] = exp2f_tab_lane(tid);

  uint32_t h0 = 0, h1 = 0;
  if (a.ring_cap) {
    h0 = a.ring_len[b];
    h1 = ring_avail(a, b, h0);
    // Decode-step mode: a finished generation is skipped (no draw).
    if (a.done && a.done[b]) {
      if (tid == 0) {
        a.out_ids[b] = a.eos_id;
        if (a.out_kept) a.out_kept[b] = 0u;
      }
      return;
    }
  } else if (a.hist && a.hist_offsets) {
    h0 = a.hist_offsets[b];
    h1 = a.hist_offsets[b + 1];
  }
  const uint32_t len_b = h0;
  const HistRow hr = hist_row(a, b, h0, h1);
  // The count table is kept current for the next step; this path counts the
  // window itself.
  if (a.ring_cap && a.counts && !counts_moved) counts_advance_all(a, b, len_b, hr.H);
  const bool use_pen = P.repetition_penalty != 1.0f && hr.H > 0;
  if (use_pen) {
    // Integer multiplicities in L2 (device-scope atomics): order-independent.
    for (uint32_t i = tid; i < V; i += kBlock)
      __hip_atomic_store(&cnt[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    for (uint32_t j = tid; j < hr.H; j += kBlock) {
      const uint32_t id = hr.at(j);
      if (id < V) atomicAdd(&cnt[id], 1u);
    }
    __syncthreads();
  }

  const bool greedy = P.temperature <= 0.0f;
  const float T = P.temperature, rp = P.repetition_penalty;
  const uint32_t n = (P.top_k > 0 && P.top_k < V) ? P.top_k : V;
  const bool sel = n < V && n <= kSelCap;  // a top-k row whose K fits the LDS list
  if (sel) {
    // Fine histogram (key bits 31..20) of the maxima of the groups of 8
    // values a thread takes at a time, for the select's bound.
    reinterpret_cast<uint4*>(L.wc)[tid] = make_uint4(0u, 0u, 0u, 0u);  // kWaves * 256 == 4 * kBlock
    __syncthreads();
  }
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  // Eight elements per thread in flight: their loads go out before any use.
  for (uint32_t i0 = tid; i0 < V; i0 += 8u * kBlock) {
    float xv[8];
    uint32_t mc[8];
    bool mo[8];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t i = i0 + u * kBlock;
      xv[u] = i < V ? row[i] : 0.0f;
      mc[u] = (use_pen && i < V) ? __hip_atomic_load(&cnt[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
      mo[u] = i < V && masked_out(a, i);
    }
    float gm = -INFINITY;  // the group's largest value (NaN never is)
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t i = i0 + u * kBlock;
      if (i >= V) break;
      float v = xv[u];
      if (mo[u]) v = -INFINITY;
      if (use_pen) v = apply_penalty(v, mc[u], rp);
      if (greedy) {
        if (v > bv) {
          bv = v;
          bi = i;
        }
      } else if (sel) {
        keysA[i] = f2key(v);  // divided later, and only where it decides (select_top_raw)
        gm = fmaxf(gm, v);
      } else {
        keysA[i] = f2key(v / T);
        idsA[i] = i;
      }
    }
    if (sel && gm > -INFINITY) atomicAdd(&L.wc[f2key(gm) >> 20], 1u);
  }
  if (greedy) {
    const uint32_t w = block_argmax(bv, bi, L.redv, L.redi);
    if (tid == 0) {
      store_result(a, b, w == 0xffffffffu ? 0u : w, len_b);
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return;
  }
  __syncthreads();
  if (sel) {
    const uint64_t* srt = select_top_raw(keysA, V, n, T, L);
    // The tail stages its terms in whichever buffer the sorted list is not in.
    float* buf = srt == L.sel ? reinterpret_cast<float*>(L.wc) : reinterpret_cast<float*>(L.sel);
    if (wave == 0) {
      draw_tail_lds(a, b, len_b, P, n, [&](uint32_t i) { return (uint32_t)(srt[i] >> 32); },
                    [&](uint32_t i) { return ~(uint32_t)srt[i]; }, a.rng_state[b], L.exptab, buf);
    }
    return;
  }
  if constexpr (!SORT) return;  // not reached: see above

  // Stable LSD radix sort, 4 x 8-bit digits, descending: ties keep
  // ascending id, which is the reference's order (generate.rs:364-367).
  // Blocks of 1024 elements are ranked in order: per wave, the lanes with
  // the same digit are found by 8 ballots; 256 threads then turn the
  // per-wave digit counts into scatter offsets (wo), so an element's
  // position is one LDS read. Eight blocks' keys and ids are loaded at a
  // time; inside a pass the barriers order LDS only (the scatter's global
  // stores are waited for at the next pass's full barrier).
  uint32_t* wo = reinterpret_cast<uint32_t*>(L.sel);  // kWaves * 256 offsets
  for (uint32_t pass = 0; pass < 4; ++pass) {
    const uint32_t shift = 8u * pass;
    const uint32_t* sK = (pass & 1) ? keysB : keysA;
    const uint32_t* sI = (pass & 1) ? idsB : idsA;
    uint32_t* dK = (pass & 1) ? keysA : keysB;
    uint32_t* dI = (pass & 1) ? idsA : idsB;
    if (tid < 256) L.bins[tid] = 0u;
    for (uint32_t i = tid; i < kWaves * 256; i += kBlock) L.wc[i] = 0u;
    __syncthreads();
    for (uint32_t i0 = tid; i0 < V; i0 += 8u * kBlock) {
      uint32_t k[8];
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) k[u] = i0 + u * kBlock < V ? sK[i0 + u * kBlock] : 0u;
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u)
        if (i0 + u * kBlock < V) atomicAdd(&L.bins[(k[u] >> shift) & 255u], 1u);
    }
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
    for (uint32_t g0 = 0; g0 < V; g0 += 8u * kBlock) {
      uint32_t kg[8], ig[8];
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        const uint32_t i = g0 + u * kBlock + tid;
        kg[u] = i < V ? sK[i] : 0u;
        ig[u] = i < V ? sI[i] : 0u;
      }
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        const uint32_t base = g0 + u * kBlock;
        if (base >= V) break;
        const bool valid = base + tid < V;
        const uint32_t k = kg[u], id = ig[u];
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
        lds_barrier();
        if (tid < 256) {
          uint32_t run = L.off[tid];
          for (uint32_t w = 0; w < kWaves; ++w) {
            const uint32_t c = L.wc[w * 256 + tid];
            wo[w * 256 + tid] = run;
            L.wc[w * 256 + tid] = 0u;
            run += c;
          }
          L.off[tid] = run;
        }
        lds_barrier();
        if (valid) {
          const uint32_t pos = wo[wave * 256 + d] + rank;
          dK[pos] = k;
          dI[pos] = id;
        }
      }
    }
    __syncthreads();  // the scatter's stores, before the next pass reads them
  }
  // Four passes end in A.
  if (wave == 0) {
    auto key_at = [&](uint32_t i) { return keysA[i]; };
    auto id_at = [&](uint32_t i) { return idsA[i]; };
    if (n <= kSelCap)
      draw_tail_lds(a, b, len_b, P, n, key_at, id_at, a.rng_state[b], L.exptab, reinterpret_cast<float*>(L.wc));
    else
      draw_tail_win(a, b, len_b, P, n, key_at, id_at, a.rng_state[b], L.exptab, reinterpret_cast<float*>(L.wc),
                    kSelCap);
  }
}

}  // namespace llmhip
