// Top-k rows of vocabularies larger than the register path holds
// (V > kMaxFastV), 0 < top_k <= kMaxFastK, temperature > 0. Row semantics:
// crates/llm-core/src/generate.rs:325-420.
//
// One persistent 1024-thread workgroup per CU takes rows j, j + grid, ...
// Each row streams through registers once, in pieces of kSPieceQ float4
// (4 per lane, 16384 values), through two register buffers:
//
//  1. the row's first two pieces are loaded at once (issued at the end of
//     the previous row, before its tail); while they land, the history's
//     multiplicities go into an LDS hash, with a bit filter so that only
//     history ids probe it.
//  2. positions past V and ids the allowed mask excludes (generate.rs:333-341:
//     their value is -inf) are set in a per-thread exclusion mask, never
//     counted or listed; ids in the history are marked, their penalty left
//     for later. Every thread counts the maxima of its groups of 8
//     unmarked values into a fine key histogram (key bits 31..20).
//  3. t0: the lower edge of the fine bin holding the K-th largest group
//     maximum. At least K values that no penalty touches lie at or above
//     it, so every value of the row's top K (after mask and penalty) does
//     too. It is lowered past the raw keys whose quotient by T ties with it
//     (division can merge values, and the reference then orders them by
//     id), and only values at or above that can be in the top K.
//  4. every value at or above the threshold is listed (value bits, id); a
//     marked value first takes its penalty (generate.rs:343-352: one step
//     per occurrence, in sequence), stopping once it is below the
//     threshold, which is exact for rp >= 1. The rest of the row streams
//     through the same two buffers, each piece's loads issued as soon as its
//     buffer is free.
//  5. the listed values are divided by T (generate.rs:357-359) into order
//     keys (value desc, id asc), ranked, and one wave runs the reference's
//     folds and the draw (draw_tail_bcast for K <= 64, draw_tail_lds
//     above), while the other waves issue the next row's loads.
//
// A row the list cannot hold (about 1.2 K values per 32768 of the row are
// listed), whose threshold is not bounded this way (fewer than K finite
// group maxima in its first two pieces, or a tie run over 64 keys), or whose
// history holds more distinct ids than the hash takes, is sampled by
// general_row in the same workgroup. Rows whose K the list cannot hold, or
// whose penalty is below 1 (it can raise a value), are not routed here
// (route_class): the sorting path's own kernel takes them.
#pragma once
#include "draw_tail.h"
#include "fast_row.h"
#include "general_row.h"
#include "sampler_common.h"
#include "wave_ops.h"

namespace llmhip {

constexpr uint32_t kSNS = 4;                 // float4 per lane and piece (two pieces in flight)
constexpr uint32_t kSPieceQ = kSNS * kBlock;  // float4 per piece
constexpr uint32_t kSCand = kStreamCand;     // listed values per row
constexpr uint32_t kSHash = 4096;            // history hash slots
constexpr uint32_t kSHashShift = 20;         // 32 - log2(kSHash)
constexpr uint32_t kSMaxDistinct = 3072;     // distinct history ids the hash takes
constexpr uint32_t kSBits = 4096;            // words of the history filter (bit id mod 2^17)
constexpr uint32_t kSEmpty = 0xffffffffu;

constexpr uint32_t kSPend = 512;             // listed values waiting for their penalty

// misc[] slots
enum : uint32_t { kSCandN = 0, kSDistinct = 1, kSFull = 2, kSPendN = 3, kSTau = 4, kSMisc = 5 };

struct StreamLds {
  __attribute__((aligned(16))) uint32_t coarse[kCoarseBins];
  __attribute__((aligned(16))) uint32_t fine[kFineBins];
  __attribute__((aligned(16))) uint64_t list[kSCand];  // (value bits, id), then order keys
  __attribute__((aligned(16))) uint64_t tmp[kSCand];   // the sort's second buffer; the tail's terms
  uint32_t hkey[kSHash];
  uint32_t hcnt[kSHash];
  uint32_t hbits[kSBits];
  uint64_t pend[kSPend];  // (raw value bits, id) of marked values at or above the threshold
  uint32_t skey[64];
  uint32_t sid[64];
  __attribute__((aligned(16))) float tail[64];
  uint64_t exptab[32];
  uint32_t misc[kSMisc];
};

union StreamKernelLds {
  StreamLds s;
  GenLds gen;  // a row handed to the sorting path
};

static_assert(2u * kSPieceQ * 4u == kStreamSpan, "the threshold's sample is the first two pieces");

// Row b's multiplicity of id (0 when absent); id's filter bit is set.
__device__ __forceinline__ uint32_t stream_count(const StreamLds& L, uint32_t id) {
  uint32_t h = (id * 2654435761u) >> kSHashShift;
  for (uint32_t probe = 0; probe < kSHash; ++probe) {
    const uint32_t k = L.hkey[h];
    if (k == id) return L.hcnt[h];
    if (k == kSEmpty) return 0u;
    h = (h + 1u) & (kSHash - 1u);
  }
  return 0u;
}

// Loads piece p of a row into buf: slot c of thread t holds float4 index
// p * kSPieceQ + c * kBlock + t (coalesced per slot). Slots past the row read
// its first float4 (a valid address); prep() marks them excluded.
// The thread's index, as a value the compiler cannot merge with another
// use: the per-slot positions derived from it are then recomputed where they
// are needed rather than held in registers across the row loop.
__device__ __forceinline__ uint32_t opaque_tid() {
  uint32_t t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((uint32_t)threadIdx.x));
  return t;
}

template <bool VEC>
__device__ __forceinline__ void stream_load(float (&buf)[kSNS * 4], const float* row, uint32_t V, uint32_t p) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const uint32_t tid = opaque_tid();
#pragma unroll
  for (int c = 0; c < (int)kSNS; ++c) {
    const uint32_t i = 4u * (p * kSPieceQ + (uint32_t)c * kBlock + tid);
    if (VEC) {
      const f4v q = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(row + (i < V ? i : 0u)));
      buf[4 * c + 0] = q.x;
      buf[4 * c + 1] = q.y;
      buf[4 * c + 2] = q.z;
      buf[4 * c + 3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) buf[4 * c + j] = __builtin_nontemporal_load(row + (i + j < V ? i + j : 0u));
    }
  }
}

// The rows of one launch (all threads). VEC: 16-byte aligned rows with a
// stride of a multiple of 4 floats (a row's last float4 may pass V, not ld).
// FULL: the call has an allowed mask or is a decode step (a ring, maybe a
// count table); the other calls run a variant compiled without that code,
// whose loop keeps fewer values live. BIGK: some row of the launch has
// K > 64; without it the kernel holds only the register rank and tail, and a
// row listing more than 512 values is handed over.
template <bool VEC, bool FULL, bool BIGK>
__device__ __forceinline__ void stream_rows(const SampleArgs& a, StreamKernelLds& U) {
  StreamLds& L = U.s;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const uint32_t V = a.V, nrows = a.launch_rows, step = gridDim.x;
  const uint32_t nq = (V + 3u) / 4u;
  // Pieces per row, rounded up to even (a piece wholly past V is read as
  // its row's first float4 and excluded): the pieces alternate between the
  // two buffers, and every row starts with piece 0 in A and piece 1 in Bf.
  const uint32_t np = ((nq + kSPieceQ - 1u) / kSPieceQ + 1u) & ~1u;
  if (tid < 32) L.exptab[tid] = exp2f_tab_lane(tid);

  // A row's scalars, fetched while the row before it is worked on and
  // before its own row loads: the loads count in order, so waiting for
  // these does not wait for the row.
  struct RowInfo {
    llmhip_params P;
    uint64_t rng0;
    uint32_t h0, h1, done;
  };
  auto row_info = [&](uint32_t rb) __attribute__((always_inline)) {
    RowInfo r;
    r.P = load_params(a, rb);
    r.rng0 = a.rng_state[rb];
    r.h0 = r.h1 = r.done = 0u;
    if (FULL && a.ring_cap) {
      r.h0 = a.ring_len[rb];
      r.h1 = ring_avail(a, rb, r.h0);
      r.done = a.done ? a.done[rb] : 0u;
    } else if (a.hist && a.hist_offsets) {
      r.h0 = a.hist_offsets[rb];
      r.h1 = a.hist_offsets[rb + 1];
    }
    return r;
  };

  float A[kSNS * 4], Bf[kSNS * 4];
  uint32_t j = blockIdx.x;
  uint32_t b = launch_row_at(a, j);
  RowInfo ri = row_info(b);
  stream_load<VEC>(A, a.logits + (size_t)b * a.ld, V, 0u);
  stream_load<VEC>(Bf, a.logits + (size_t)b * a.ld, V, 1u);

  while (true) {
    const uint32_t jn = j + step;
    const uint32_t bn = jn < nrows ? launch_row_at(a, jn) : b;
    const RowInfo ri_next = row_info(bn);
    const float* row = a.logits + (size_t)b * a.ld;
    const llmhip_params P = ri.P;
    const uint32_t K = P.top_k;
    const float T = P.temperature, rp = P.repetition_penalty;
    const uint64_t rng0 = ri.rng0;
    // 0: sampled here; 1: handed over to the sorting path; 3: nothing to do
    // (a row of another launch, or a finished generation).
    uint32_t outcome = 0u;
    // A row of another launch (a mixed call without the class table).
    if (!a.row_cls_on && !(route_class(P, V) & a.row_class_mask)) outcome = 3u;

    const uint32_t len_b = ri.h0;
    const HistRow hr = FULL ? hist_row(a, b, ri.h0, ri.h1)
                            : HistRow{a.hist + ri.h0, 0u, 0u, ri.h1 > ri.h0 ? ri.h1 - ri.h0 : 0u};
    LLMHIP_MARK(0);
    if (outcome == 0u && ri.done) {
      // Decode-step mode: a finished generation is skipped (no draw).
      if (tid == 0) {
        a.out_ids[b] = a.eos_id;
        if (a.out_kept) a.out_kept[b] = 0u;
      }
      outcome = 3u;
    }
    // The count table is kept current for the next step; this path counts
    // the window itself.
    bool counts_moved = false;
    if (FULL && outcome == 0u && a.ring_cap && a.counts) {
      counts_advance_all(a, b, len_b, hr.H);
      counts_moved = true;
    }
    const bool use_pen = rp != 1.0f && hr.H > 0u;

    if (outcome == 0u) {
      // 1. History multiplicities (order-independent integer LDS atomics)
      //    and the filter; the histogram and counters start at zero.
      for (uint32_t i = tid; i < kFineBins; i += kBlock) L.fine[i] = 0u;
      if (tid < kSMisc) L.misc[tid] = 0u;
      if (use_pen) {
        for (uint32_t s = tid; s < kSHash; s += kBlock) {
          L.hkey[s] = kSEmpty;
          L.hcnt[s] = 0u;
        }
        for (uint32_t s = tid; s < kSBits; s += kBlock) L.hbits[s] = 0u;
      }
      lds_barrier();
      if (use_pen) {
        for (uint32_t q = tid; q < hr.H; q += kBlock) {
          const uint32_t id = hr.at(q);
          if (id >= V) continue;
          atomicOr(&L.hbits[(id >> 5) & (kSBits - 1u)], 1u << (id & 31u));
          uint32_t h = (id * 2654435761u) >> kSHashShift;
          for (uint32_t probe = 0; probe < kSHash; ++probe) {
            const uint32_t old = atomicCAS(&L.hkey[h], kSEmpty, id);
            if (old == id || old == kSEmpty) {
              if (old == kSEmpty && atomicAdd(&L.misc[kSDistinct], 1u) >= kSMaxDistinct) L.misc[kSFull] = 1u;
              atomicAdd(&L.hcnt[h], 1u);
              break;
            }
            h = (h + 1u) & (kSHash - 1u);
          }
        }
        lds_barrier();
        if (L.misc[kSFull]) outcome = 1u;
      }
      LLMHIP_MARK(1);
    }

    // 2. Mask, bounds and marks, as bit masks over the 16 values a thread
    //    holds in a buffer (the values themselves stay as loaded): xm, set
    //    past V and where the allowed mask excludes the id (-inf in the
    //    reference, so never listed); pm, set for ids in the history. Then
    //    the group maxima of the values in neither.
    const bool masked = FULL && (a.allowed || a.allowed_bits);
    auto prep = [&](uint32_t p, uint32_t& xm) __attribute__((always_inline)) -> uint32_t {
      const uint32_t tid = opaque_tid();
      uint32_t pm = 0u;
      xm = 0u;
      const bool last = (p + 1u) * kSPieceQ * 4u > V;  // the piece holds positions past V
#pragma unroll
      for (int c = 0; c < (int)kSNS; ++c) {
        const uint32_t i0 = 4u * (p * kSPieceQ + (uint32_t)c * kBlock + tid);
        if (use_pen && i0 < V) pm |= ((L.hbits[(i0 >> 5) & (kSBits - 1u)] >> (i0 & 31u)) & 15u) << (4 * c);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t i = i0 + (uint32_t)q;
          if ((last && i >= V) || (masked && i < V && masked_out(a, i))) xm |= 1u << (4 * c + q);
        }
      }
      return pm;
    };
    auto gmax = [&](const float (&buf)[kSNS * 4], uint32_t skip) __attribute__((always_inline)) {
      // A wave none of whose values is skipped (no mask, no history id)
      // takes plain maxima.
      const bool any_skip = __ballot(skip != 0u) != 0ull;
#pragma unroll
      for (int c = 0; c < (int)kSNS; c += 2) {
        float g = -INFINITY;
        if (!any_skip) {
#pragma unroll
          for (int e = 4 * c; e < 4 * c + 8; ++e) g = fmaxf(g, buf[e]);
        } else {
#pragma unroll
          for (int e = 4 * c; e < 4 * c + 8; ++e)
            if (!((skip >> e) & 1u)) g = fmaxf(g, buf[e]);
        }
        if (g > -INFINITY) atomicAdd(&L.fine[f2key(g) >> 20], 1u);
      }
    };
    float tf = 0.0f;
    // 4. Values at or above tf listed: unmarked ones by a wave scan of the
    //    per-thread counts, marked ones (rare) after their penalty, each
    //    taking a slot of its own.
    auto list_piece = [&](const float (&buf)[kSNS * 4], uint32_t p, uint32_t pm, uint32_t xm)
                          __attribute__((always_inline)) {
      const uint32_t tid = opaque_tid();
      // The compares as one bit mask, then the exclusions and marks as
      // whole-mask operations.
      uint32_t ge = 0u;
#pragma unroll
      for (int e = 0; e < (int)kSNS * 4; ++e) ge |= (buf[e] >= tf ? 1u : 0u) << e;
      ge &= ~xm;
      const uint32_t hits = ge & ~pm, pen = ge & pm;
      const uint32_t hc = (uint32_t)__popc(hits);
      const uint32_t inc = wave_incl_scan(hc);
      const uint32_t wt = readlane_u32(inc, 63);
      uint32_t base = 0u;
      if (wt != 0u) {
        if (lane == 0) base = atomicAdd(&L.misc[kSCandN], wt);
        base = readlane_u32(base, 0);
      }
      // A thread holds a hit or two at most, as a rule: one pass per hit,
      // the value picked out of the buffer by selects (a register array
      // takes constant indices only).
      uint32_t o = base + inc - hc;
      for (uint32_t h = hits; h != 0u; h &= h - 1u) {
        const uint32_t e = (uint32_t)__builtin_ctz(h);
        float v = buf[0];
#pragma unroll
        for (int q = 1; q < (int)kSNS * 4; ++q) v = e == (uint32_t)q ? buf[q] : v;
        const uint32_t i = 4u * (p * kSPieceQ + (e >> 2) * kBlock + tid) + (e & 3u);
        if (o < kSCand) L.list[o] = ((uint64_t)__float_as_uint(v) << 32) | i;
        ++o;
      }
      // Marked values wait in their own list: their penalty is applied once
      // the row is streamed (a penalty loop here would weigh on every
      // piece's code).
      for (uint32_t h = pen; h != 0u; h &= h - 1u) {
        const uint32_t e = (uint32_t)__builtin_ctz(h);
        float v = buf[0];
#pragma unroll
        for (int q = 1; q < (int)kSNS * 4; ++q) v = e == (uint32_t)q ? buf[q] : v;
        const uint32_t i = 4u * (p * kSPieceQ + (e >> 2) * kBlock + tid) + (e & 3u);
        const uint32_t q = atomicAdd(&L.misc[kSPendN], 1u);
        if (q < kSPend) L.pend[q] = ((uint64_t)__float_as_uint(v) << 32) | i;
      }
    };

    uint32_t n = 0u;
    bool fetched = false;  // the next row's first two pieces are out
    if (outcome == 0u) {
      uint32_t xmA, xmB;
      uint32_t pmA = prep(0u, xmA);
      uint32_t pmB = prep(1u, xmB);
      gmax(A, pmA | xmA);
      gmax(Bf, pmB | xmB);
      LLMHIP_MARK(2);
      lds_barrier();
      coarse_from_fine(L.fine, L.coarse);
      lds_barrier();
      // 3. The threshold, selected by one wave (ahead of the others on its
      //    SIMD) and published in LDS; 1 says the row is not bounded.
      if (wave == 0u) {
        __builtin_amdgcn_s_setprio(3);
        const uint32_t t0 = hist_locate(L.coarse, L.fine, K, lane).lo;
        const uint32_t t = t0 ? lower_past_ties(t0, T, lane) : 0u;
        (void)lds_publish(&L.misc[kSTau], t ? t : 1u);
        __builtin_amdgcn_s_setprio(0);
      }
      const uint32_t tpub = lds_wait_nonzero(&L.misc[kSTau], 1u, a);
      const uint32_t tlo = tpub > 1u ? tpub : 0u;
      LLMHIP_MARK(3);
      if (tlo == 0u) {
        outcome = 1u;
      } else {
        tf = key2f(tlo);
        // Pieces p (in A) and p + 1 (in Bf); each buffer reloads as soon as
        // it is listed, with the piece two ahead or, past this row's last,
        // with the next row's first two pieces (they land during this row's
        // rank and tail).
        for (uint32_t p = 0u; p < np; p += 2u) {
          if (p > 0u) pmA = prep(p, xmA);
          list_piece(A, p, pmA, xmA);
          if (p == 0u) LLMHIP_MARK(10);
          if (p + 2u < np) {
            stream_load<VEC>(A, row, V, p + 2u);
          } else if (jn < nrows) {
            stream_load<VEC>(A, a.logits + (size_t)bn * a.ld, V, 0u);
            LLMHIP_MARK(9);
          }
          if (p == 0u) LLMHIP_MARK(11);
          if (p > 0u) pmB = prep(p + 1u, xmB);
          list_piece(Bf, p + 1u, pmB, xmB);
          if (p == 0u) LLMHIP_MARK(4);
          if (p + 3u < np) {
            stream_load<VEC>(Bf, row, V, p + 3u);
          } else if (jn < nrows) {
            stream_load<VEC>(Bf, a.logits + (size_t)bn * a.ld, V, 1u);
          }
        }
        fetched = true;
        LLMHIP_MARK(5);
        lds_barrier();
        // The marked values' penalties (generate.rs:343-352), stopping once
        // a value is below the threshold (exact for rp >= 1).
        const uint32_t npend = L.misc[kSPendN];
        if (npend != 0u) {
          if (npend > kSPend) {
            outcome = 1u;
          } else {
            for (uint32_t q = tid; q < npend; q += kBlock) {
              const uint64_t r = L.pend[q];
              const uint32_t i = (uint32_t)r;
              const float v = apply_penalty_above(__uint_as_float((uint32_t)(r >> 32)), stream_count(L, i), rp, tf);
              if (v >= tf) {
                const uint32_t o = atomicAdd(&L.misc[kSCandN], 1u);
                if (o < kSCand) L.list[o] = ((uint64_t)__float_as_uint(v) << 32) | i;
              }
            }
            lds_barrier();
          }
        }
        n = L.misc[kSCandN];
        // At least K: the K group maxima above t0 are listed.
        // (A launch without BIGK never holds K > 64; that test only keeps
        // its 64-entry rank output in bounds.)
        if (n > (BIGK ? kSCand : 512u) || n < K || (!BIGK && K > 64u)) outcome = 1u;
      }
    }

    if (outcome == 1u) {
      // The sorting path, in this workgroup (its LDS overlaps this path's).
      if (tid == 0) atomicAdd(a.handovers, 1u);
      __syncthreads();
      general_row<false>(a, b, U.gen, counts_moved);
      __syncthreads();
      if (tid < 32) L.exptab[tid] = exp2f_tab_lane(tid);
    } else if (outcome == 0u) {
      // 5. Order keys, rank, tail.
      for (uint32_t i = tid; i < n; i += kBlock) {
        const uint64_t r = L.list[i];
        L.list[i] = cand_order(f2key(__uint_as_float((uint32_t)(r >> 32)) / T), (uint32_t)r);
      }
      lds_barrier();
      LLMHIP_MARK(12);
      if (!BIGK || (K <= 64u && n <= 512u)) {
        if (n <= 128u) {
          rank_in_regs<2>(L.list, n, K, wave, lane, L.skey, L.sid);
        } else if (n <= 256u) {
          rank_in_regs<4>(L.list, n, K, wave, lane, L.skey, L.sid);
        } else {
          rank_in_regs<8>(L.list, n, K, wave, lane, L.skey, L.sid);
        }
        lds_barrier();
        LLMHIP_MARK(6);
        if (wave == 0) {
          uint64_t st_next = rng0;
          const float u = next_f32(st_next);
          draw_tail_bcast(a, b, len_b, P, K, lane < K ? L.skey[lane] : kKeyNone, lane < K ? L.sid[lane] : 0u, u,
                          st_next, L.exptab, L.tail);
          LLMHIP_MARK(7);
        }
      } else if constexpr (BIGK) {
        const uint64_t* srt = n <= kBlock        ? sort_desc_lds<1>(L.list, L.tmp, n)
                              : n <= 2u * kBlock ? sort_desc_lds<2>(L.list, L.tmp, n)
                                                 : sort_desc_lds<4>(L.list, L.tmp, n);
        float* buf = reinterpret_cast<float*>(srt == L.list ? L.tmp : L.list);
        auto key_at = [&](uint32_t i) { return (uint32_t)(srt[i] >> 32); };
        auto id_at = [&](uint32_t i) { return ~(uint32_t)srt[i]; };
        stage_exp_terms(buf, K, key_at, L.exptab, tid, kBlock);
        lds_barrier();
        if (wave == 0) draw_tail_lds<true>(a, b, len_b, P, K, key_at, id_at, rng0, L.exptab, buf);
      }
    }
    if (jn >= nrows) break;
    // The next row's first two pieces, where not out yet (a row this path
    // did not list).
    if (!fetched) {
      stream_load<VEC>(A, a.logits + (size_t)bn * a.ld, V, 0u);
      stream_load<VEC>(Bf, a.logits + (size_t)bn * a.ld, V, 1u);
    }
    ri = ri_next;
    LLMHIP_MARK(8);
    j = jn;
    b = bn;
  }
}

}  // namespace llmhip
