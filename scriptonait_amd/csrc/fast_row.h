// Register path of the gfx950 sampler: one row per 1024-thread workgroup,
// V <= 32768, 0 < top_k <= 4096 (and greedy rows).
//
// Row semantics: crates/llm-core/src/generate.rs:325-420. The row is read
// once from HBM into registers, all of it at once (the memory queues run
// full from the first cycle), and the selection threshold is taken from the
// waves whose data lands first, so only a compare, one settle pass, two
// workgroup barriers, a rank over ~1.5K candidates and the sequential tail
// remain after the last byte lands.
//
// Layout. Lane l of wave w holds chunk c = floats 4l..4l+3 of the 1 KiB
// block c*16 + w of the row, loaded with one nontemporal dwordx4: every
// load is 1 KiB contiguous per wave, and the blocks of any set of waves are
// spread evenly over the whole row.
//
// Per wave:
//  1. the row lands: per-chunk and per-thread maxima.
//  2. the first kTauWaves (8) waves to get here put their per-thread maxima
//     in a two-level key histogram; the 8th selects the threshold (about
//     1.6K of the row's values expected at or above it, scaled from the half
//     of the row those waves hold) and publishes it in LDS.
//  3. the first 7 of them count the history ids: u16 multiplicities and
//     per-owner masks of penalized slots, integer LDS atomics whose result
//     does not depend on order (in count-table mode the first wave slides
//     the row's table in HBM instead).
//  4. each chunk whose maximum reaches the threshold is compared value by
//     value; hits go to the wave's LDS region.
//  5. the wave settles its hits (mask, penalty m times in sequence,
//     recheck, one division by T) into the candidate list.
//  6. barrier; the count check (>= K proves the threshold); rank; barrier.
//  7. one wave replays the reference's folds and draws.
//
// Selecting on raw values is exact: the mask sets -inf and a penalty
// p >= 1 never raises a value (l/p <= l for l > 0, l*p <= l for l <= 0,
// each correctly rounded), so every value at or above the threshold after
// mask and penalty was at or above it before. Rows with p < 1 (or NaN) take
// the general path.
#pragma once
#include <cstddef>
#include <type_traits>

#include "draw_tail.h"
#include "sampler_common.h"
#include "wave_ops.h"

// Profiling hooks: a profiling build defines LLMHIP_MARK(i) (a timestamp
// per wave at phase i) and LLMHIP_NOTE(i, v) (a recorded value); both are
// empty otherwise.
#ifndef LLMHIP_MARK
#define LLMHIP_MARK(i)
#endif
#ifndef LLMHIP_NOTE
#define LLMHIP_NOTE(i, v)
#endif

namespace llmhip {

// LDS needed by the general path (about 53 KB).
struct GenLds {
  uint32_t bins[256];
  uint32_t off[256];
  __attribute__((aligned(16))) uint32_t wc[kWaves * 256];  // also the tail's terms (<= kSelCap floats)
  float redv[kWaves];
  uint32_t redi[kWaves];
  uint64_t exptab[32];
  uint64_t sel[kSelCap];  // the K selected order keys (key << 32 | ~id)
  uint32_t sv[4];         // select state
};

constexpr uint32_t kFastCand = 2048;              // candidates per row
constexpr uint32_t kEntries = 64;                 // scan entries per wave
constexpr uint32_t kCoarseBins = 256;             // key bits 31..24
constexpr uint32_t kFineBins = 4096;              // key bits 31..20
constexpr uint32_t kTauWaves = 8;                 // waves whose maxima form the threshold sample
constexpr uint32_t kSpecNum = 8, kSpecDen = 5;    // the threshold aims at ~(kSpecNum/kSpecDen)*K values
constexpr uint32_t kSpecMaxK = 384;               // larger K: the scan entries would overflow; proven threshold
constexpr uint32_t kRefineCount = 16;             // a fine bin holding more keys is split once more
constexpr uint32_t kSortedK = 1024;               // K up to which the sorted top K is copied to skey/sid
constexpr uint32_t kBigCand = 7168;               // K > kSortedK: candidates per row (the scan entries' LDS)

// misc[] slots
constexpr int kSyncSample = 0;  // sample waves in the histogram (bits 20+) and the positions they hold
constexpr int kSyncHist = 1;    // waves whose history ids are counted
constexpr int kCandN = 2;       // candidates in ord[]
constexpr int kOverflow = 3;    // some wave's region overflowed
constexpr int kTauState = 4;    // 0: not yet, 1: row not bounded here, else the threshold key
constexpr int kArrive = 6;   // waves whose row has landed, in arrival order
constexpr int kSampled = 7;  // row positions held by the sample waves (for a second pass)
constexpr int kSyncZero = 8; // waves whose share of the count table is zeroed
constexpr int kGreedyMax = 9; // greedy rows: key of the row's largest value known without a penalty
constexpr int kCandN2 = 10;    // candidates of the second speculative pass
constexpr int kOverflow2 = 11; // some wave's region overflowed in it
constexpr int kTau2 = 12;      // its threshold key (1: no second pass)
constexpr int kTau0 = 13;      // the proven threshold key (1: not bounded here)

// BIGK: the large-K kernel's scan entries hold 128 per wave (a proven
// threshold for K up to 1024 puts about 1.2 K chunks in them).
// K > kSortedK: the candidate list takes the LDS of the scan entries
// (ent, etag and ord, which are contiguous), and its sort ping-pongs with
// big_tmp, which the count table's LDS holds once the penalties are applied.
template <int NCH, bool BIGK = false>
struct FastLds {
  static constexpr uint32_t kEnt = BIGK ? 128u : kEntries;
  union {
    uint32_t cnt[NCH * 2048];  // u16 history multiplicities, two per word (V <= NCH*4096)
    GenLds gen;                // the general path's LDS when a row falls back
    uint64_t big_tmp[BIGK ? kBigCand : 1];
  };
  uint32_t pm[kBlock];  // per-thread mask: slot is penalized
  __attribute__((aligned(16))) uint32_t coarse[kCoarseBins];
  __attribute__((aligned(16))) uint32_t fine[kFineBins];
  float4 ent[kWaves * kEnt];  // scan entries: a lane's 4 values of a chunk with a hit
  __attribute__((aligned(16))) uint32_t etag[kWaves * kEnt];  // chunk position | chunk << 28
  __attribute__((aligned(16))) uint64_t ord[kFastCand];  // settled order keys; then the tail's terms
  uint32_t skey[kSortedK];  // sorted top-K: post-temperature key
  uint32_t sid[kSortedK];   //               id
  uint64_t exptab[32];
  __attribute__((aligned(16))) float tail[128];
  float redv[kWaves];
  uint32_t redi[kWaves];
  uint32_t misc[16];
};

// The large-K candidate list: kBigCand order keys over ent, etag and ord.
template <int NCH>
__device__ __forceinline__ uint64_t* big_list(FastLds<NCH, true>& L) {
  using F = FastLds<NCH, true>;
  static_assert(offsetof(F, etag) == offsetof(F, ent) + sizeof(L.ent) &&
                    offsetof(F, ord) == offsetof(F, etag) + sizeof(L.etag) &&
                    sizeof(L.ent) + sizeof(L.etag) + sizeof(L.ord) >= kBigCand * sizeof(uint64_t),
                "ent, etag and ord hold the large-K list");
  return reinterpret_cast<uint64_t*>(L.ent);
}

// Read-only inputs that every lane of a wave reads at the same address go
// through the constant address space, so they become scalar (SMEM) loads:
// those count on lgkmcnt and never queue behind the row's vector loads.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* as_const(const T* p) {
  return (const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ llmhip_params load_params(const SampleArgs& a, uint32_t b) {
  llmhip_params P = a.shared;
  if (a.params) {
    const auto* q = as_const(a.params) + (size_t)b * a.params_stride;
    P.temperature = q->temperature;
    P.top_k = q->top_k;
    P.top_p = q->top_p;
    P.min_p = q->min_p;
    P.repetition_penalty = q->repetition_penalty;
  }
  return P;
}

__device__ __forceinline__ float apply_penalty(float v, uint32_t m, float rp) {
  // generate.rs:343-352, once per occurrence, in sequence.
  for (; m; --m) v = v > 0.0f ? v / rp : v * rp;
  return v;
}

// The same, for a caller that only asks whether the result reaches `floor`
// (and uses the value only when it does): with rp >= 1 every step can only
// lower the value (v / rp <= v for v > 0, v * rp <= v otherwise, each
// correctly rounded) or turn it into NaN, so once it is below floor the
// result is below floor (or NaN) whatever the remaining steps do, and the
// loop stops there. A history that repeats a top candidate's id many times
// otherwise runs one dependent division per occurrence.
__device__ __forceinline__ float apply_penalty_above(float v, uint32_t m, float rp, float floor) {
  for (; m && !(v < floor); --m) v = v > 0.0f ? v / rp : v * rp;
  return v;
}

__device__ __forceinline__ bool masked_out(const SampleArgs& a, uint32_t id) {
  // generate.rs:333-341
  if (id >= a.allowed_len || id == a.eos_id) return false;
  if (a.allowed) return a.allowed[id] == 0;
  return a.allowed_bits && ((a.allowed_bits[id >> 5] >> (id & 31u)) & 1u) == 0u;
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

// Workgroup barrier that orders LDS only: outstanding global loads stay in
// flight across it (a full __syncthreads would wait for every row load).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One wave announces that its LDS writes so far are complete (LDS-only
// release: no wait on the wave's outstanding global loads). Returns the
// number of waves that had signalled before, in every lane.
__device__ __forceinline__ uint32_t lds_signal(uint32_t* ctr) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  uint32_t before = 0u;
  if ((threadIdx.x & 63u) == 0u) before = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return readlane_u32(before, 0);
}

__device__ __forceinline__ uint32_t lds_peek(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Wait until *ctr >= target. Every wave that counts toward a target signals
// it unconditionally before it waits on anything, so the wait ends. The
// spin is bounded all the same (a.spin_limit spins, about 0.1 s by
// default): should that ever run out (a bug, not an input condition), the
// wave records it in the call's status word and carries on, so the kernel
// still finishes and the failure is reported instead of the GPU hanging.
__device__ __forceinline__ void lds_wait(const uint32_t* ctr, uint32_t target, const SampleArgs& a) {
  uint32_t spins = 0;
  while (lds_peek(ctr) < target) {
    if (++spins > a.spin_limit) {
      if ((threadIdx.x & 63u) == 0u) atomicOr(a.status, kStatusSyncTimeout);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Publish v (nonzero) in *p unless a value is there already; returns the
// value *p holds afterwards (the first one published wins).
__device__ __forceinline__ uint32_t lds_publish(uint32_t* p, uint32_t v) {
  uint32_t old = 0u;  // the value expected: nothing published yet
  if ((threadIdx.x & 63u) == 0u)
    __hip_atomic_compare_exchange_strong(p, &old, v, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  // On success old still holds 0; on failure it holds the value found.
  old = readlane_u32(old, 0);
  return old ? old : v;
}

// Wait until *p != 0 and return that value. Should the bounded spin run out
// (as in lds_wait), the wave publishes `fallback` itself, so every wave of
// the workgroup still reads one and the same value.
__device__ __forceinline__ uint32_t lds_wait_nonzero(uint32_t* p, uint32_t fallback, const SampleArgs& a) {
  uint32_t spins = 0, v;
  while ((v = lds_peek(p)) == 0u) {
    if (++spins > a.spin_limit) {
      if ((threadIdx.x & 63u) == 0u) atomicOr(a.status, kStatusSyncTimeout);
      v = lds_publish(p, fallback);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  return v;
}

#ifndef LLMHIP_STRIDED
#define LLMHIP_STRIDED 1
#endif
// Block (1 KiB, 256 floats) that wave `wave` holds as its chunk c.
template <int NCH>
__device__ __forceinline__ uint32_t chunk_block(uint32_t c, uint32_t wave) {
  return LLMHIP_STRIDED ? c * kWaves + wave : wave * NCH + c;
}
// Row position of chunk c's first float in lane `lane` of wave `wave`.
template <int NCH>
__device__ __forceinline__ uint32_t chunk_pos(uint32_t c, uint32_t wave, uint32_t lane) {
  return (chunk_block<NCH>(c, wave) * 64u + lane) * 4u;
}
// Thread (wave*64 + lane) and slot (4*chunk + j) holding row position p.
template <int NCH>
__device__ __forceinline__ uint32_t pos_owner(uint32_t p) {
  return (LLMHIP_STRIDED ? (p >> 8) % kWaves : (p >> 8) / NCH) * 64u + ((p >> 2) & 63u);
}
template <int NCH>
__device__ __forceinline__ uint32_t pos_slot(uint32_t p) {
  return (LLMHIP_STRIDED ? (p >> 8) / kWaves : (p >> 8) % NCH) * 4u + (p & 3u);
}
// Row positions (< V) held by wave `wave`.
template <int NTOT, int NCH>
__device__ __forceinline__ uint32_t wave_positions(uint32_t wave, uint32_t V) {
  uint32_t n = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const uint32_t s0 = chunk_block<NTOT>((uint32_t)c, wave) * 256u;
    n += s0 >= V ? 0u : min(256u, V - s0);
  }
  return n;
}

// Candidate order key: larger = earlier in the reference's sort (value
// desc, then id asc, generate.rs:364-367).
__device__ __forceinline__ uint64_t cand_order(uint32_t wkey, uint32_t id) {
  return ((uint64_t)wkey << 32) | (uint64_t)(0xffffffffu - id);
}

// f(integral_constant<int, I>) for I = I0 .. N-1, expanded at compile time
// (chunk indices must be constants: the row lives in registers).
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Lane i < 32 gets kExp2fTab[i] from instruction immediates: no memory
// access, so the table never waits behind the row's loads.
__device__ __forceinline__ uint64_t exp2f_tab_lane(uint32_t lane) {
  uint64_t v = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) v = lane == (uint32_t)i ? kExp2fTab[i] : v;
  return v;
}

// Where the Q-th largest key counted in the two-level histogram (coarse:
// key bits 31..24, fine: bits 31..20) lies: lo, the lower edge of the fine
// bin holding it (0 when fewer than Q keys were counted), cnt, that bin's
// count, and need (1..cnt), its rank inside the bin. Wave-local.
struct HistPos {
  uint32_t lo, cnt, need;
};
__device__ __forceinline__ HistPos hist_locate(const uint32_t* coarse, const uint32_t* fine, uint32_t Q,
                                               uint32_t lane) {
  // Lane l holds coarse bins 255-4l .. 252-4l (w, z, y, x: descending).
  const uint4 q = reinterpret_cast<const uint4*>(coarse)[63u - lane];
  const uint32_t lt = q.x + q.y + q.z + q.w;
  const uint32_t ci = wave_incl_scan(lt);
  const uint64_t lm = __ballot(Q <= ci);
  if (!lm) return HistPos{0u, 0u, 0u};
  const uint32_t l = (uint32_t)__ffsll((unsigned long long)lm) - 1u;
  uint32_t need = Q - (readlane_u32(ci, l) - readlane_u32(lt, l));
  const uint32_t cw = readlane_u32(q.w, l), cz = readlane_u32(q.z, l), cy = readlane_u32(q.y, l);
  uint32_t cb = 255u - 4u * l;
  if (need > cw) {
    need -= cw;
    --cb;
    if (need > cz) {
      need -= cz;
      --cb;
      if (need > cy) {
        need -= cy;
        --cb;
      }
    }
  }
  // Lanes 0..15 hold the 16 fine bins of coarse bin cb, descending.
  const uint32_t fc = lane < 16u ? fine[cb * 16u + 15u - lane] : 0u;
  const uint32_t fi = wave_incl_scan(fc);
  const uint64_t fm = __ballot(lane < 16u && need <= fi);
  const uint32_t fl = (uint32_t)__ffsll((unsigned long long)fm) - 1u;
  const uint32_t cnt = readlane_u32(fc, fl);
  return HistPos{(cb * 16u + 15u - fl) << 20, cnt, need - (readlane_u32(fi, fl) - cnt)};
}

// The coarse histogram as sums of the fine one (coarse bin c = fine bins
// 16c .. 16c+15), for histograms counted into fine bins only: their keys
// crowd a few coarse bins, whose atomics would serialize. All threads; a
// barrier must follow before hist_locate reads it.
__device__ __forceinline__ void coarse_from_fine(const uint32_t* fine, uint32_t* coarse) {
  static_assert(kFineBins == 4u * kBlock && kFineBins == 16u * kCoarseBins, "one uint4 per thread");
  const uint32_t tid = threadIdx.x;
  const uint4 q = reinterpret_cast<const uint4*>(fine)[tid];
  uint32_t v = q.x + q.y + q.z + q.w;
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  if ((tid & 3u) == 0u) coarse[tid >> 2] = v;
}

// The Q-th largest key counted in the histogram, as a key threshold. exact:
// the lower edge of the fine bin holding it, so at least Q counted keys lie
// at or above the result. Otherwise an estimate inside that bin, taking its
// keys as evenly spread. Returns 0 when fewer than Q keys were counted.
__device__ __forceinline__ uint32_t hist_select(const uint32_t* coarse, const uint32_t* fine, uint32_t Q,
                                                bool exact, uint32_t lane) {
  const HistPos h = hist_locate(coarse, fine, Q, lane);
  if (exact || h.lo == 0u) return h.lo;
  // need <= cnt <= 1024, so need << 20 fits in 32 bits.
  return h.lo + (1u << 20) - (h.need << 20) / (h.cnt + 1u);
}

// Lower a raw-value key threshold past every key whose value divided by T
// ties with it (division can merge distinct values, and the reference then
// orders the merged ones by id). Lane l tests the key l+1 below; runs of
// ties are at most ceil(2T)+1 keys long, so 64 covers T < 31. Returns 0
// when the row is not bounded this way (threshold at or below -inf, or a
// longer run).
__device__ __forceinline__ uint32_t lower_past_ties(uint32_t tau, float T, uint32_t lane) {
  if (tau <= 0x007fffffu + 64u) return 0u;
  const uint32_t wt = f2key(key2f(tau) / T);
  const uint64_t ties = __ballot(f2key(key2f(tau - 1u - lane) / T) == wt);
  const uint64_t run = ~ties;
  if (run == 0ull) return 0u;
  const uint32_t lo = tau - ((uint32_t)__ffsll((unsigned long long)run) - 1u);
  return lo > 0x007fffffu ? lo : 0u;
}

// Ranks of the n candidates in ord[] (order keys, all distinct): rank(i) =
// #{j : ord_j > ord_i}; the K best are written to skey/sid in sorted order.
// All 16 waves share the candidates;
// each wave holds the whole list in registers (NR keys per lane) and ranks
// an even slice of it, two at a time, one ballot per held key. Lane i
// collects candidate i's rank, so the loop body touches no LDS and waits on
// nothing.
template <int NR>
__device__ __forceinline__ void rank_in_regs(const uint64_t* ord, uint32_t n, uint32_t K, uint32_t wave,
                                             uint32_t lane, uint32_t* skey, uint32_t* sid) {
  uint64_t oj[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    const uint32_t j = lane + 64u * t;
    oj[t] = j < n ? ord[j] : 0ull;
  }
  const uint32_t per = (n + kWaves - 1) / kWaves;  // <= 4 * NR
  const uint32_t i0 = min(n, wave * per), cnt = min(n, i0 + per) - i0;
  const uint64_t mi = lane < cnt ? ord[i0 + lane] : 0ull;
  uint32_t myr = 0xffffffffu;
  for (uint32_t i = 0; i < cnt; i += 2u) {
    const uint64_t oa = readlane_u64(mi, i), ob = readlane_u64(mi, min(i + 1u, cnt - 1u));
    uint32_t ra = 0u, rb = 0u;
#pragma unroll
    for (int t = 0; t < NR; ++t) {
      ra += (uint32_t)__popcll((unsigned long long)__ballot(oj[t] > oa));
      rb += (uint32_t)__popcll((unsigned long long)__ballot(oj[t] > ob));
    }
    myr = lane == i ? ra : lane == i + 1u ? rb : myr;
  }
  if (lane < cnt && myr < K) {
    skey[myr] = (uint32_t)(mi >> 32);
    sid[myr] = 0xffffffffu - (uint32_t)mi;
  }
}

// Sorts v[0, n) descending in place (all threads of the workgroup): a
// bitonic network over N = the power of two >= n, with v[n, N) set to 0,
// which sorts last (every order key here is above 0). v holds at least N
// entries. The order keys are distinct, so the order is the total one.
__device__ __forceinline__ void bitonic_sort_desc(uint64_t* v, uint32_t n) {
  const uint32_t tid = threadIdx.x;
  uint32_t N = 1u;
  while (N < n) N <<= 1;
  for (uint32_t i = n + tid; i < N; i += kBlock) v[i] = 0ull;
  lds_barrier();
  for (uint32_t k = 2u; k <= N; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0u; j >>= 1) {
      for (uint32_t p = tid; p < N / 2u; p += kBlock) {
        const uint32_t i = ((p & ~(j - 1u)) << 1) | (p & (j - 1u));  // bit j of i clear
        const uint64_t x = v[i], y = v[i | j];
        if ((i & k) == 0u ? x < y : x > y) {
          v[i] = y;
          v[i | j] = x;
        }
      }
      lds_barrier();
    }
  }
}

// Sorts the n order keys in ord[] descending (all threads of the
// workgroup; ord and tmp hold n rounded up to 64 entries). Runs of 64 keys
// are sorted in registers, one key per lane, by a bitonic network of lane
// exchanges (no barrier); then runs are merged in pairs, log2(n / 64)
// rounds between ord and tmp with one barrier each. In a round, thread t
// writes the E merged keys at positions tE .. tE+E-1 (E * 1024 >= n and E a
// power of two, so they lie in one pair of runs A, B): a binary search along
// its diagonal of the merge (the merge path) finds how many of the keys
// before them come from A, then E steps merge from the two heads. A key of
// A goes before an equal key of B (only the zero padding has equal keys).
// Returns the buffer that holds the sorted keys (ord or tmp), past a
// barrier.
template <int E>
__device__ __forceinline__ uint64_t* sort_desc_lds(uint64_t* ord, uint64_t* tmp, uint32_t n) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t np = (n + 63u) & ~63u;
  for (uint32_t r = wave; r * 64u < np; r += kWaves) {
    const uint32_t i = r * 64u + lane;
    uint64_t x = i < n ? ord[i] : 0ull;
    for (uint32_t k = 2u; k <= 64u; k <<= 1) {
      for (uint32_t j = k >> 1; j > 0u; j >>= 1) {
        const uint64_t y = __shfl_xor(x, (int)j, 64);
        const bool keep_max = ((lane & k) == 0u) == ((lane & j) == 0u);
        x = keep_max ? (x > y ? x : y) : (x < y ? x : y);
      }
    }
    ord[i] = x;
  }
  lds_barrier();
  uint64_t* src = ord;
  uint64_t* dst = tmp;
  const uint32_t g = tid * (uint32_t)E;  // this thread's first output position
  for (uint32_t R = 64u; R < np; R <<= 1) {
    if (g < np) {
      const uint32_t s0 = g & ~(2u * R - 1u);
      const uint32_t la = min(R, np - s0), lb = min(2u * R, np - s0) - la;
      const uint64_t* A = src + s0;
      const uint64_t* B = A + la;
      const uint32_t d = g - s0;
      // The first d outputs are A[0, i) and B[0, d - i): i is the first
      // index whose A key does not go before B[d - i - 1].
      uint32_t lo = d > lb ? d - lb : 0u, hi = min(d, la);
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (A[mid] >= B[d - mid - 1u]) {
          lo = mid + 1u;
        } else {
          hi = mid;
        }
      }
      uint32_t ia = lo, jb = d - lo;
      uint64_t ha = ia < la ? A[ia] : 0ull, hb = jb < lb ? B[jb] : 0ull;
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const bool take_a = jb >= lb || (ia < la && ha >= hb);
        dst[g + (uint32_t)k] = take_a ? ha : hb;
        if (k + 1 < E) {
          if (take_a) {
            ++ia;
            ha = ia < la ? A[ia] : 0ull;
          } else {
            ++jb;
            hb = jb < lb ? B[jb] : 0ull;
          }
        }
      }
    }
    lds_barrier();
    uint64_t* t = src;
    src = dst;
    dst = t;
  }
  return src;
}

// More candidates than the register ranks hold (n <= kFastCand): sort them
// and write the K best to skey/sid in sorted order.
__device__ __forceinline__ void rank_in_lds(uint64_t* ord, uint64_t* tmp, uint32_t n, uint32_t K, uint32_t* skey,
                                            uint32_t* sid) {
  static_assert(kFastCand <= 2u * kBlock, "two keys per thread");
  const uint64_t* src = n <= kBlock ? sort_desc_lds<1>(ord, tmp, n) : sort_desc_lds<2>(ord, tmp, n);
  for (uint32_t i = threadIdx.x; i < K; i += kBlock) {
    const uint64_t o = src[i];
    skey[i] = (uint32_t)(o >> 32);
    sid[i] = 0xffffffffu - (uint32_t)o;
  }
}

// One row on the register path. Returns false (uniformly across the
// workgroup, before writing any output) when the row needs the general
// path.
// GREEDY: the launch takes the greedy rows (temperature <= 0) only, else
// the top-k rows only; each variant is compiled without the other's code.
// CMODE: a decode step with a count table (a.ring and a.counts set); the
// other calls run variants compiled without the table's code.
// BIGK: some top-k row of the call has K > 64. Without it the kernel holds
// only the small-K rank and tail (a smaller kernel), and a row with more
// than 512 candidates goes to the general path.
template <int NCH, bool VEC, bool GREEDY, bool CMODE, bool BIGK>
__device__ __forceinline__ bool fast_row(const SampleArgs& a, FastLds<NCH, BIGK>& L) {
  constexpr uint32_t kEnt = FastLds<NCH, BIGK>::kEnt;
  static_assert(sizeof(FastLds<NCH, BIGK>) <= 160u * 1024u, "LDS");
  static_assert(NCH * 4 <= 32, "slot masks are 32 bits");
  typedef float f4v __attribute__((ext_vector_type(4)));

  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const uint32_t V = a.V;
  // The kernel arguments this path reads, fetched here in one batch (left
  // to itself the compiler fetches some at their first use, behind the
  // row's loads, and the LDS barrier below would wait for them).
  asm volatile("" ::"s"(a.logits), "s"(a.ld), "s"(a.V), "s"(a.params), "s"(a.params_stride), "s"(a.hist),
               "s"(a.hist_offsets), "s"(a.slotmask), "s"(a.status), "s"(a.rng_state), "s"(a.out_ids),
               "s"(a.out_probs), "s"(a.out_kept), "s"(a.row_class_mask), "s"(a.ring), "s"(a.ring_len),
               "s"(a.done), "s"(a.ring_cap), "s"(a.window), "s"(a.hist_start), "s"(a.spin_limit));
  asm volatile("" ::"s"(a.shared.temperature), "s"(a.shared.top_k), "s"(a.shared.top_p), "s"(a.shared.min_p),
               "s"(a.shared.repetition_penalty), "s"(a.eos_id), "s"(a.allowed), "s"(a.allowed_len), "s"(a.B),
               "s"(a.scratch), "s"(a.scratch_row_words), "s"(a.row_cls_on));
  const uint32_t b = launch_row(a);
  LLMHIP_MARK(0);

  // Every global load below is issued unconditionally (positions past V and
  // absent inputs read a valid dummy address), so each wait in the compiled
  // code names exactly the loads it needs. A wave's loads complete at a
  // limited rate (a CU holds only part of its 128 KiB row in flight, and a
  // wave stalls at a load until earlier data has returned), so every wave
  // issues its part of the row as early as it can: the first two chunks,
  // the LDS set-up and its barrier in their shadow, then the rest. The
  // history ids are fetched later, by the first waves whose rows are in.
  //
  // The row's scalars go out first, by vector loads (lane l reads word l),
  // which count in order with the row's loads: a scalar load would share its
  // counter with LDS operations, and every LDS wait before it returned
  // (behind the row) would wait for it.
  // hv: lanes 0-1 read hist_offsets[b], [b+1] (CSR), or lanes 0-4 read
  // ring_len[b], done[b], hist_start[b], counted[2b], counted[2b+1]
  // (decode-step mode; the last two with a count table).
  const bool ring = a.ring_cap != 0u;
  const bool has_hist = ring || (a.hist_offsets && a.hist);
  constexpr bool cmode = CMODE;  // multiplicities from the count table
  const uint32_t l7 = lane & 7u;
  const uint32_t* hvsrc = ring ? (l7 == 1u && a.done ? a.done + b
                                  : l7 == 2u && a.hist_start ? a.hist_start + b
                                  : (l7 == 3u || l7 == 4u) && cmode ? a.counted + 2u * b + (l7 - 3u)
                                  : a.ring_len + b)
                               : (has_hist ? a.hist_offsets + b + (lane & 1u) : a.slotmask);
  const uint32_t hv = *hvsrc;
  const uint32_t rv = reinterpret_cast<const uint32_t*>(a.rng_state + b)[lane & 1u];
  const uint32_t pw =
      a.params ? reinterpret_cast<const uint32_t*>(a.params + (size_t)b * a.params_stride)[min(lane, 4u)] : 0u;
  const uint32_t mkbits = a.slotmask[tid];  // masked-out slots (allowed mask), or 0
  __builtin_amdgcn_sched_barrier(0);

  const float* row = a.logits + (size_t)b * a.ld;
  float x[NCH * 4];
  auto load_chunk = [&](int c) __attribute__((always_inline)) {
    const uint32_t base = chunk_pos<NCH>((uint32_t)c, wave, lane);
    if (VEC) {
      const f4v q = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(row + (base < V ? base : 0u)));
      x[4 * c + 0] = q.x;
      x[4 * c + 1] = q.y;
      x[4 * c + 2] = q.z;
      x[4 * c + 3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * c + j] = __builtin_nontemporal_load(row + (base + j < V ? base + j : 0u));
    }
  };
  constexpr int NB0 = NCH >= 2 ? 2 : 1;
#pragma unroll
  for (int c = 0; c < NB0; ++c) load_chunk(c);
  __builtin_amdgcn_sched_barrier(0);

  // LDS set-up; every wave zeroes its share of the count table later.
  if (wave == 0 && lane < 32) L.exptab[lane] = exp2f_tab_lane(lane);
  reinterpret_cast<uint4*>(L.fine)[tid] = make_uint4(0u, 0u, 0u, 0u);  // kFineBins / 4 == kBlock
  if (tid < kCoarseBins / 4) reinterpret_cast<uint4*>(L.coarse)[tid] = make_uint4(0u, 0u, 0u, 0u);
  L.pm[tid] = 0u;
  if (tid < 16) L.misc[tid] = 0u;
  lds_barrier();  // LDS tables are zeroed
  LLMHIP_MARK(1);
#pragma unroll
  for (int c = NB0; c < NCH; ++c) load_chunk(c);
  __builtin_amdgcn_sched_barrier(0);

  const uint32_t hv0 = readlane_u32(hv, 0), hv1 = readlane_u32(hv, 1), hv2 = readlane_u32(hv, 2);
  const uint32_t hv3 = readlane_u32(hv, 3), hv4 = readlane_u32(hv, 4);
  const uint32_t h0 = has_hist ? hv0 : 0u;
  // CSR: hist_offsets[b + 1]; ring: the ring's tokens still in the cache.
  const uint32_t h1 = ring ? (a.hist_start ? (hv0 > hv2 ? hv0 - hv2 : 0u) : hv0) : (has_hist ? hv1 : 0u);
  const bool row_done = ring && a.done && hv1 != 0u;
  const uint32_t len_b = h0;  // ring length (decode-step mode)
  const uint64_t rng0 = ((uint64_t)readlane_u32(rv, 1) << 32) | readlane_u32(rv, 0);
  llmhip_params P = a.shared;
  if (a.params) {
    P.temperature = __uint_as_float(readlane_u32(pw, 0));
    P.top_k = readlane_u32(pw, 1);
    P.top_p = __uint_as_float(readlane_u32(pw, 2));
    P.min_p = __uint_as_float(readlane_u32(pw, 3));
    P.repetition_penalty = __uint_as_float(readlane_u32(pw, 4));
  }
  const float T = P.temperature, rp = P.repetition_penalty;
  const HistRow hr = hist_row(a, b, h0, h1);
  const uint32_t H = rp != 1.0f ? hr.H : 0u;
  const bool use_pen = H > 0 && H < 65536u;
  // This wave's share of the count table (only when a history may be used).
  if (a.hist) {
    uint4* c4 = reinterpret_cast<uint4*>(L.cnt);
    for (uint32_t i = tid; i < (V + 7u) / 8u; i += kBlock) c4[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  lds_signal(&L.misc[kSyncZero]);
  // The uniform draw of this row, ahead of the tail (rng.rs:16-34).
  uint64_t st_next = rng0;
  const float u_draw = next_f32(st_next);

  // Positions past V (in the one chunk that straddles V, or in chunks
  // wholly past it) become -inf before their first use: no value at or
  // above a threshold, never a maximum. The test is uniform per wave.
  auto prep = [&](int c) __attribute__((always_inline)) {
    if ((chunk_block<NCH>((uint32_t)c, wave) + 1u) * 256u > V) {
      const uint32_t base = chunk_pos<NCH>((uint32_t)c, wave, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * c + j] = base + j < V ? x[4 * c + j] : -INFINITY;
    }
  };

  const uint32_t cls = row_class(P, V);
  if (!(cls & a.row_class_mask)) return true;
  // Decode-step mode: a finished generation is skipped (no draw).
  if (row_done) {
    if (tid == 0) {
      a.out_ids[b] = a.eos_id;
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return true;
  }
  // The count table's change for this step (every later return hands the
  // row over with the table done). A rebuild takes the whole workgroup (it
  // waits for the row's loads; it happens on a generation's first step and
  // after a cache reset); a slide is made below by the first wave to land.
  const CountsPlan cplan = cmode ? counts_plan(a, hv3, hv4, len_b, hr.H) : CountsPlan{0u, 0u, 0u, 0u, false};
  if (cmode && cplan.rebuild) {
    counts_rebuild(a, b, cplan);  // ends published, past a barrier
    if (wave == 0) lds_signal(&L.misc[kSyncHist]);
  }
  // Rows handed over from here on have had their count table moved (the
  // sorting path does not move it again).
  auto slide_before_handover = [&]() __attribute__((always_inline)) {
    if (cmode && !cplan.rebuild && wave == 0) counts_slide(a, b, cplan);
  };
  if (__builtin_expect(H >= 65536u, 0)) {  // a u16 multiplicity could overflow
    slide_before_handover();
    return false;
  }
  // A penalty below 1 (or NaN) can raise a value above the raw one, so the
  // selection on raw values below does not bound such rows.
  if (!GREEDY && use_pen && !(rp >= 1.0f)) {
    slide_before_handover();
    return false;
  }
  const uint32_t K = P.top_k;  // 0 < K < V, K <= kMaxFastK unless greedy (row class)
  // More than skey/sid hold: the candidates are listed over the scan
  // entries' LDS, sorted there, and the tail reads the K best in place.
  const bool huge = BIGK && K > kSortedK;

  // Multiplicity of position p in the window. Positions past V (padding
  // slots) have none, and the table holds no word for them.
  auto count_of = [&](uint32_t p) __attribute__((always_inline)) {
    if (cmode) return p < V ? counts_at(a, b, p) : 0u;
    return (L.cnt[p >> 1] >> ((p & 1u) << 4)) & 0xffffu;
  };
  auto add_hist = [&](uint32_t id) __attribute__((always_inline)) {
    if (id < V) {
      const uint32_t sh = (id & 1u) << 4;
      const uint32_t old = atomicAdd(&L.cnt[id >> 1], 1u << sh);
      if (((old >> sh) & 0xffffu) == 0u) atomicOr(&L.pm[pos_owner<NCH>(id)], 1u << pos_slot<NCH>(id));
    }
  };
  // History multiplicities (integer LDS atomics: the counts do not depend on
  // the order). The first occurrence of an id marks its slot in the owner
  // thread's mask. Waves part = 0 .. nparts-1 share the ids, 8 per lane in
  // flight at a time.
  auto count_history = [&](uint32_t part, uint32_t nparts) __attribute__((always_inline)) {
    if (use_pen) {
      lds_wait(&L.misc[kSyncZero], kWaves, a);
      const uint32_t stride = nparts * 64u;
      for (uint32_t j0 = part * 64u; j0 < H; j0 += 8u * stride) {
        uint32_t ids[8];
#pragma unroll
        for (uint32_t u = 0; u < 8u; ++u) {
          const uint32_t j = j0 + u * stride + lane;
          ids[u] = j < H ? hr.at(j) : 0xffffffffu;
        }
#pragma unroll
        for (uint32_t u = 0; u < 8u; ++u) add_hist(ids[u]);  // ids >= V are ignored
      }
    }
    lds_signal(&L.misc[kSyncHist]);
  };
  // Mask and penalty of this thread's slot e, in the reference's order.
  // floor: a value that falls below it can no longer matter (-inf: none).
  auto fix_value = [&](float v, int e, uint32_t pmv, float floor) __attribute__((always_inline)) {
    if ((mkbits >> e) & 1u) v = -INFINITY;
    if ((pmv >> e) & 1u)
      v = apply_penalty_above(v, count_of(chunk_pos<NCH>((uint32_t)(e >> 2), wave, lane) + (e & 3)), rp, floor);
    return v;
  };
  auto fix_all = [&](uint32_t pmv, float floor) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if ((((pmv | mkbits) >> (4 * c)) & 0xfu) != 0u) {
#pragma unroll
        for (int j = 0; j < 4; ++j) x[4 * c + j] = fix_value(x[4 * c + j], 4 * c + j, pmv, floor);
      }
    }
  };
  // Count-table mode: this thread's slots whose id is in the window (after
  // the step's change is published). A chunk's four ids are two table
  // words; positions past V have none.
  auto table_bits = [&]() __attribute__((always_inline)) {
    const uint32_t* row = counts_row(a, b);
    constexpr int G = NCH < 4 ? NCH : 4;  // chunks whose words are in flight together
    uint32_t bits = 0u;
#pragma unroll
    for (int c0 = 0; c0 < NCH; c0 += G) {
      uint32_t wd[2 * G];
#pragma unroll
      for (int c = 0; c < G; ++c) {
        const uint32_t p0 = chunk_pos<NCH>((uint32_t)(c0 + c), wave, lane);
        wd[2 * c] = p0 < V ? __hip_atomic_load(&row[p0 >> 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        wd[2 * c + 1] =
            p0 + 2u < V ? __hip_atomic_load(&row[(p0 >> 1) + 1u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
      }
#pragma unroll
      for (int e = 0; e < G * 4; ++e) {
        const uint32_t p = chunk_pos<NCH>((uint32_t)(c0 + (e >> 2)), wave, lane) + (uint32_t)(e & 3);
        const uint32_t m = (wd[e >> 1] >> ((e & 1) << 4)) & 0xffffu;
        if (m != 0u && p < V) bits |= 1u << (4 * c0 + e);
      }
    }
    return bits;
  };
  // With rp >= 1 a penalty only lowers a value (v / rp for v > 0, v * rp
  // otherwise), and a slot outside the history (or masked) has its final
  // value already. So `known`, the thread's maximum over those slots, is a
  // lower bound on its final maximum that needs no penalty.
  auto known_max = [&](uint32_t pmv) __attribute__((always_inline)) {
    float kv = -INFINITY;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e)
      if ((((pmv | mkbits) >> e) & 1u) == 0u) kv = fmaxf(kv, x[e]);
    return kv;
  };

  if constexpr (GREEDY) {
    // ops/loss.rs:6-16 over the masked, penalized row (before temperature).
#pragma unroll
    for (int c = 0; c < NCH; ++c) prep(c);
    uint32_t pmv = 0u;
    if (cmode) {
      // The table names the penalized slots once the step's change is in.
      if (!cplan.rebuild && wave == 0) {
        counts_slide(a, b, cplan);
        counts_publish();
        lds_signal(&L.misc[kSyncHist]);
      }
      lds_wait(&L.misc[kSyncHist], 1u, a);
      if (use_pen) pmv = table_bits();
    } else {
      count_history(wave, kWaves);
      if (use_pen) {
        lds_wait(&L.misc[kSyncHist], kWaves, a);
        pmv = L.pm[tid];
      }
    }
    if (use_pen && rp >= 1.0f) {
      // The row's largest known value M0 bounds the winner from below: a
      // history slot whose raw value is below M0 can neither win nor tie
      // (a tie goes to the lower position), so only the others are
      // penalized; the rest keep their raw values, which lose all the same.
      const uint32_t kk = wave_max_u32(f2key(known_max(pmv)));
      if (lane == 0u) atomicMax(&L.misc[kGreedyMax], kk);
      lds_barrier();
      const float m0 = key2f(L.misc[kGreedyMax]);
      uint32_t need = 0u;
#pragma unroll
      for (int e = 0; e < NCH * 4; ++e)
        if (x[e] >= m0) need |= 1u << e;
      // A value pushed below M0 loses too, so its penalty stops there.
      fix_all(pmv & need, m0);
    } else {
      fix_all(pmv, -INFINITY);  // rp < 1 raises values: every step counts
    }
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) {
      if (x[e] > bv) {
        bv = x[e];
        bi = chunk_pos<NCH>((uint32_t)(e >> 2), wave, lane) + (e & 3);
      }
    }
    const uint32_t w = block_argmax(bv, bi, L.redv, L.redi);
    if (tid == 0) {
      store_result(a, b, w == 0xffffffffu ? 0u : w, len_b);
      if (a.out_kept) a.out_kept[b] = 0u;
    }
    return true;
  }
  // 1. The row has landed: per-chunk and per-thread maxima (NaN is never a
  //    maximum).
  constexpr int NS = NCH;
  auto max4 = [&](int c) __attribute__((always_inline)) {
    return fmaxf(fmaxf(x[4 * c], x[4 * c + 1]), fmaxf(x[4 * c + 2], x[4 * c + 3]));
  };
  float mc[NCH];
  float tm = -INFINITY;
#pragma unroll
  for (int c = 0; c < NS; ++c) {
    prep(c);
    mc[c] = max4(c);
    tm = fmaxf(tm, mc[c]);
  }
  LLMHIP_MARK(2);

  // The sample position the speculative threshold takes: the target
  // (kSpecNum/kSpecDen)*K scaled to the positions the sample holds.
  auto spec_q = [&](uint32_t sampled) __attribute__((always_inline)) {
    // In 32 bits: sampled <= kTauWaves * 2048 and K <= kMaxFastK.
    static_assert((uint64_t)kSpecNum * kMaxFastK * kTauWaves * 2048u + kSpecDen * kMaxFastV < (1ull << 32), "fits");
    return (kSpecNum * K * sampled + kSpecDen * V - 1u) / (kSpecDen * V) + 2u;
  };
  // 2. The first kTauWaves waves to get here put their sample maxima in the
  //    histogram, and the last of them selects the speculative threshold:
  //    the Q-th largest sampled maximum, with Q scaled from the target
  //    (kSpecNum/kSpecDen)*K to the positions the sample holds.
  uint32_t arrive = 0u;
  if (lane == 0u) arrive = __hip_atomic_fetch_add(&L.misc[kArrive], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  arrive = readlane_u32(arrive, 0);
  {
    if (arrive < kTauWaves) {
      if (tm > -INFINITY) {  // a NaN or -inf maximum is not counted
        const uint32_t k = f2key(tm);
        bin_add_grouped(L.coarse, k >> 24);
        atomicAdd(&L.fine[k >> 20], 1u);
      }
      // kSyncSample counts the sample waves in bits 20 and up and the row
      // positions they hold below (at most kTauWaves * 2048): the last
      // wave's own atomic returns the sample's size.
      const uint32_t pos = wave_positions<NCH, NS>(wave, V);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      uint32_t before = 0u;
      if (lane == 0u)
        before = __hip_atomic_fetch_add(&L.misc[kSyncSample], (1u << 20) + pos, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_WORKGROUP);
      before = readlane_u32(before, 0);
      if ((before >> 20) == kTauWaves - 1u) {
        const uint32_t sampled = (before & 0xfffffu) + pos;
        if (lane == 0u) L.misc[kSampled] = sampled;  // for a second pass
        // Every other wave waits for this one-wave chain: it takes the
        // issue slots of its SIMD first (wave priority, reset below).
        __builtin_amdgcn_s_setprio(3);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        LLMHIP_MARK(3);
        const uint32_t tkey = K <= kSpecMaxK ? lower_past_ties(hist_select(L.coarse, L.fine, spec_q(sampled), false, lane), T, lane) : 0u;
        // A bounded threshold key is above 0x007fffff (lower_past_ties), so
        // 1 is free to say "not bounded".
        (void)lds_publish(&L.misc[kTauState], tkey ? tkey : 1u);
        __builtin_amdgcn_s_setprio(0);
      }
    }
  }
  // The history counts, by the first kTauWaves - 1 waves (the last sample
  // wave selects the threshold instead): their ids are fetched while the
  // other waves' rows are still landing, and counted while they wait for
  // the threshold, so the waves whose rows land last find the counts done.
  if (cmode) {
    // The first wave to land slides the count table and announces it once
    // its atomics are complete in L2.
    if (!cplan.rebuild && arrive == 0u) {
      counts_slide(a, b, cplan);
      counts_publish();
      lds_signal(&L.misc[kSyncHist]);
    }
  } else if (arrive < kTauWaves - 1u) {
    count_history(arrive, kTauWaves - 1u);
  }

  // 3. The scan: every lane whose maximum over a chunk reaches the
  //    published threshold appends one entry (the chunk's 4 values and its
  //    position) to the wave's region: one compare per chunk, and for the
  //    chunks where some lane hits, one ballot offset and two LDS writes.
  const uint32_t tau = lds_wait_nonzero(&L.misc[kTauState], 1u, a);
  // Not bounded by the sample (a large K, or a long run of ties after the
  // division by T): the proven threshold below takes the row. Every wave
  // read the same published state.
  const bool spec = tau > 1u;
  float tf = key2f(tau);
  LLMHIP_MARK(4);
  uint32_t nent = 0u;  // this wave's entries
  auto scan_chunk = [&](int c, float mcv) __attribute__((always_inline)) {
    const bool hit = mcv >= tf;
    const uint64_t m = __ballot(hit);
    if (m) {
      const uint32_t o = nent + lanes_below(m);
      if (hit && o < kEnt) {
        L.ent[wave * kEnt + o] = make_float4(x[4 * c], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]);
        L.etag[wave * kEnt + o] = chunk_pos<NCH>((uint32_t)c, wave, lane) | ((uint32_t)c << 28);
      }
      nent += (uint32_t)__popcll((unsigned long long)m);
    }
  };
  if (spec) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) scan_chunk(c, mc[c]);
  }
  LLMHIP_MARK(5);

  // 5. Settle this wave's entries: each lane takes an entry and handles its
  //    hits one at a time (almost always one): mask, penalty, recheck,
  //    then the post-temperature order key (one
  //    division, generate.rs:357-359), appended to ord[] with one LDS
  //    atomic per round.
  uint32_t pmv = 0u;
  uint32_t slot_n = kCandN, slot_o = kOverflow;  // the pass's candidate count and overflow flag
  auto settle = [&]() __attribute__((always_inline)) {
    if (__builtin_expect(nent > kEnt, 0)) {
      if (lane == 0) atomicOr(&L.misc[slot_o], 1u);
      return;
    }
    for (uint32_t k0 = 0; k0 < nent; k0 += 64u) {
      const uint32_t k = k0 + lane;
      float4 ev = make_float4(0.f, 0.f, 0.f, 0.f);
      uint32_t tag = 0u;
      if (k < nent) {
        ev = L.ent[wave * kEnt + k];
        tag = L.etag[wave * kEnt + k];
      }
      const uint32_t base = tag & 0x00ffffffu, c = tag >> 28;
      uint32_t rem = k < nent ? ((ev.x >= tf ? 1u : 0u) | (ev.y >= tf ? 2u : 0u) | (ev.z >= tf ? 4u : 0u) |
                                 (ev.w >= tf ? 8u : 0u))
                              : 0u;
      // The entry's owner is a lane of this wave: fetch its mask words.
      const uint32_t owner = pos_owner<NCH>(base);
      const uint32_t mkown = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((owner & 63u) << 2), (int)mkbits);
      const uint32_t pmown = (!use_pen || k >= nent) ? 0u : cmode ? 0xffffffffu : L.pm[owner];
      while (__ballot(rem != 0u)) {
        // A lane takes part in a round only while it has a hit left.
        bool ok = rem != 0u;
        const uint32_t j = ok ? (uint32_t)__builtin_ctz(rem) : 0u;
        rem &= rem - 1u;
        float v = j == 0 ? ev.x : j == 1 ? ev.y : j == 2 ? ev.z : ev.w;
        const uint32_t e = 4u * c + j, pos = base + j;
        if (ok) {
          if ((mkown >> e) & 1u) v = -INFINITY;
          if ((pmown >> e) & 1u) v = apply_penalty_above(v, count_of(pos), rp, tf);
          ok = v >= tf;
        }
        const uint64_t mk = __ballot(ok);
        if (mk) {
          uint32_t o = 0u;
          if (lane == 0) o = atomicAdd(&L.misc[slot_n], (uint32_t)__popcll((unsigned long long)mk));
          o = readlane_u32(o, 0) + lanes_below(mk);
          if (ok && o < kFastCand) L.ord[o] = cand_order(f2key(v / T), pos);
        }
      }
    }
  };
  if (cmode) {
    lds_wait(&L.misc[kSyncHist], 1u, a);
    if (use_pen) pmv = 0xffffffffu;
  } else if (use_pen) {
    lds_wait(&L.misc[kSyncHist], kTauWaves - 1u, a);
    pmv = L.pm[tid];
  }
  settle();
  lds_barrier();
  LLMHIP_MARK(6);
  uint32_t n = L.misc[kCandN];
  bool ovf = L.misc[kOverflow] != 0u;
  LLMHIP_NOTE(12, n);
  // A speculative threshold the penalty undercut (a history holding the
  // row's own top ids): once more from the sample histogram, at a position
  // deep enough for the 5K/4 - n survivors still missing (at most 8 times
  // the first). One wave selects it (a selection in every wave would compete
  // for the ALUs).
  if (__builtin_expect(spec && n < K && !ovf, 0)) {
    if (wave == 0u) {
      __builtin_amdgcn_s_setprio(3);  // as for the first threshold
      const uint64_t q = spec_q(L.misc[kSampled]);
      // q sample positions stand for (kSpecNum/kSpecDen)*K values; the
      // values below the first threshold are assumed to survive the penalty
      // two times in three, so 3/2 * (5K/4 - n) more of them are wanted.
      const uint64_t need = 5u * K / 4u - n;  // n < K
      const uint64_t want = q + (q * need * 3u * kSpecDen + 2u * kSpecNum * K - 1u) / (2u * kSpecNum * K);
      const uint64_t q2 = want < 8u * q ? want : 8u * q;
      const uint32_t tk2 = lower_past_ties(hist_select(L.coarse, L.fine, (uint32_t)q2, false, lane), T, lane);
      (void)lds_publish(&L.misc[kTau2], tk2 != 0u && key2f(tk2) < tf ? tk2 : 1u);
      __builtin_amdgcn_s_setprio(0);
    }
    const uint32_t tk2 = lds_wait_nonzero(&L.misc[kTau2], 1u, a);
    const bool again = tk2 > 1u;
    if (again) {
      LLMHIP_NOTE(13, 4u);
      LLMHIP_MARK(11);
      tf = key2f(tk2);
      nent = 0u;
      slot_n = kCandN2;
      slot_o = kOverflow2;
#pragma unroll
      for (int c = 0; c < NCH; ++c) scan_chunk(c, mc[c]);
      LLMHIP_MARK(12);
      settle();
      LLMHIP_MARK(13);
    }
    lds_barrier();  // the pass is settled, and every wave is past the histogram reads
    if (again) {
      n = L.misc[kCandN2];
      ovf = L.misc[kOverflow2] != 0u;
      LLMHIP_NOTE(15, n);
    }
  }
  // The small-K kernel ranks at most 512 candidates.
  const uint32_t ncap = BIGK ? kFastCand : 512u;
  if (__builtin_expect(!spec || n < K || n > ncap || ovf, 0)) {
    LLMHIP_NOTE(13, spec ? 1u : 2u);
    // The proven threshold. Known values are those of the slots outside the
    // history and the mask: final without a penalty, which (rp >= 1) only
    // lowers a value. t0 is the lower edge of the fine bin holding the K-th
    // largest of the 1024 per-thread known maxima (or per-chunk maxima), so
    // at least K known values lie at or above it, and a history slot can
    // reach it only if its raw value does. The scan and settle run again at t0 (lowered past
    // ties after the division by T): at least K candidates. Everyone is past
    // the sample histogram and the scan entries, so their LDS is reused.
    const uint32_t pmr = cmode && use_pen ? table_bits() : pmv;
    const uint32_t known = ~(pmr | mkbits);
    // A large K takes the K-th largest of the 8192 per-chunk known maxima
    // instead: 1024 per-thread maxima put far more than K values above
    // their K-th largest when K is a large share of 1024.
    const bool by_chunk = BIGK && K > kSpecMaxK;
    // The histograms below count into fine bins only (coarse_from_fine).
    reinterpret_cast<uint4*>(L.fine)[tid] = make_uint4(0u, 0u, 0u, 0u);
    lds_barrier();  // every wave has read the candidate count and overflow flag above
    LLMHIP_MARK(11);
    if (tid == 0) {
      L.misc[kCandN] = 0u;
      L.misc[kOverflow] = 0u;
    }
    slot_n = kCandN;
    slot_o = kOverflow;
    if (by_chunk) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        float cm = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if ((known >> (4 * c + j)) & 1u) cm = fmaxf(cm, x[4 * c + j]);
        if (cm > -INFINITY) atomicAdd(&L.fine[f2key(cm) >> 20], 1u);
      }
    } else {
      const float tm = known_max(pmr);
      if (tm > -INFINITY) atomicAdd(&L.fine[f2key(tm) >> 20], 1u);
    }
    lds_barrier();
    coarse_from_fine(L.fine, L.coarse);
    lds_barrier();
    // A finite maximum's key is at least 0x00800000, above -inf's and NaN's
    // (hist_locate's 0 says fewer than K threads hold a known value).
    if (wave == 0u) {
      __builtin_amdgcn_s_setprio(3);  // as for the first threshold
      const uint32_t t0 = hist_locate(L.coarse, L.fine, K, lane).lo;
      // A large K goes to the per-slot narrowing below, which needs only
      // some key at or below its K-th largest known value: t0, or, when
      // fewer than K chunks hold a known value, the lowest finite key.
      const uint32_t tk = huge ? (t0 ? t0 : 0x00800000u) : t0 ? lower_past_ties(t0, T, lane) : 0u;
      (void)lds_publish(&L.misc[kTau0], tk ? tk : 1u);
      __builtin_amdgcn_s_setprio(0);
    }
    const uint32_t tk0 = lds_wait_nonzero(&L.misc[kTau0], 1u, a);
    if (tk0 <= 1u) return false;
    LLMHIP_MARK(12);
    tf = key2f(tk0);
    // A large K puts more values at or above t0 than the scan entries hold.
    if (!huge) {
      nent = 0u;
#pragma unroll
      for (int c = 0; c < NCH; ++c) scan_chunk(c, mc[c]);
      settle();
      lds_barrier();
      LLMHIP_MARK(13);
      n = L.misc[kCandN];
    }
    if (__builtin_expect(huge || n > ncap || L.misc[kOverflow] != 0u, 0)) {
      // Too many values at or above the threshold for the scan entries or
      // the list (a large K): narrow it per slot. Level 1: the fine bin
      // holding the K-th largest known value at or above it (tk0 <= t0, so
      // at least K are). Level 2, when that bin is
      // crowded: 12 more key bits inside it. At least K final values lie at
      // or above the result.
      LLMHIP_NOTE(13, 3u);
      uint32_t* fine1 = reinterpret_cast<uint32_t*>(L.ent);  // kWaves * kEnt float4 >= kFineBins words
      uint32_t* coarse1 = L.etag;                              // kWaves * kEnt words >= kCoarseBins
      reinterpret_cast<uint4*>(fine1)[tid] = make_uint4(0u, 0u, 0u, 0u);
      lds_barrier();  // every wave has read the count and flag, and is past the entries
      // (A fresh copy of the mask per loop: shared between the loops, its 32
      // per-slot bits would stay live in registers from one to the next.)
      uint32_t kn1 = known;
      asm volatile("" : "+v"(kn1));
#pragma unroll
      for (int e = 0; e < NCH * 4; ++e) {
        const uint32_t k = f2key(x[e]);
        if (((kn1 >> e) & 1u) && k >= tk0) atomicAdd(&fine1[k >> 20], 1u);
      }
      lds_barrier();  // level 1 counted; every wave is past level 0's reads
      coarse_from_fine(fine1, coarse1);
      lds_barrier();
      const HistPos h1 = hist_locate(coarse1, fine1, K, lane);
      LLMHIP_NOTE(14, h1.cnt);
      uint32_t thr = h1.lo;
      if (h1.cnt > kRefineCount) {
        reinterpret_cast<uint4*>(L.fine)[tid] = make_uint4(0u, 0u, 0u, 0u);
        lds_barrier();
        uint32_t kn2 = known;
        asm volatile("" : "+v"(kn2));
#pragma unroll
        for (int e = 0; e < NCH * 4; ++e) {
          const uint32_t k = f2key(x[e]);
          if (((kn2 >> e) & 1u) && (k >> 20) == (h1.lo >> 20)) atomicAdd(&L.fine[(k << 12) >> 20], 1u);
        }
        lds_barrier();
        coarse_from_fine(L.fine, L.coarse);
        lds_barrier();
        thr = h1.lo | (hist_locate(L.coarse, L.fine, h1.need, lane).lo >> 12);
      }
      const uint32_t tkey = lower_past_ties(thr, T, lane);
      if (tkey == 0u) return false;
      LLMHIP_MARK(14);
      tf = key2f(tkey);
      uint64_t* list = L.ord;
      uint32_t lcap = kFastCand;
      if constexpr (BIGK) {
        if (huge) {
          lds_barrier();  // every wave is past the level-1 bins, which the list overwrites
          list = big_list(L);
          lcap = kBigCand;
        }
      }
      // Every thread's final values at or above the threshold, then their
      // places in the list from a scan of the per-thread counts (a counter
      // in LDS would serialize the waves' appends, one per slot).
      uint32_t hits = 0u;
#pragma unroll
      for (int e = 0; e < NCH * 4; ++e) {
        float v = x[e];
        bool ok = v >= tf && ((mkbits >> e) & 1u) == 0u;
        if (ok && ((pmr >> e) & 1u)) {
          v = apply_penalty_above(v, count_of(chunk_pos<NCH>((uint32_t)(e >> 2), wave, lane) + (uint32_t)(e & 3)), rp,
                                  tf);
          ok = v >= tf;
        }
        x[e] = v;
        hits |= (ok ? 1u : 0u) << e;
      }
      const uint32_t hc = (uint32_t)__popc(hits);
      const uint32_t hinc = wave_incl_scan(hc);
      if (lane == 63u) L.redi[wave] = hinc;
      lds_barrier();
      uint32_t o = hinc - hc, total = 0u;
#pragma unroll
      for (uint32_t w = 0; w < kWaves; ++w) {
        const uint32_t t = L.redi[w];
        o += w < wave ? t : 0u;
        total += t;
      }
      // Listed as (value bits, position) first: the division by T is then
      // made once per listed value, spread over all threads, instead of by
      // every wave for each slot where one of its lanes has a hit.
#pragma unroll
      for (int e = 0; e < NCH * 4; ++e) {
        if ((hits >> e) & 1u) {
          const uint32_t pos = chunk_pos<NCH>((uint32_t)(e >> 2), wave, lane) + (uint32_t)(e & 3);
          if (o < lcap) list[o] = ((uint64_t)__float_as_uint(x[e]) << 32) | pos;
          ++o;
        }
      }
      lds_barrier();
      for (uint32_t i = tid; i < min(total, lcap); i += kBlock) {
        const uint64_t r = list[i];
        list[i] = cand_order(f2key(__uint_as_float((uint32_t)(r >> 32)) / T), (uint32_t)r);
      }
      lds_barrier();
      LLMHIP_MARK(15);
      n = total;
    }
    // Heavy ties or an unusually flat top: not bounded by the register path.
    if (n < K || n > (huge ? kBigCand : ncap)) return false;
  }

  // 6. Ranks by (w key desc, id asc).
  LLMHIP_MARK(9);
  if constexpr (BIGK) {
    if (huge) {
      // The list sorted in LDS (the count table's LDS is free once every
      // penalty is applied); the tail stages its terms in the other buffer.
      static_assert(kBigCand <= 8u * kBlock, "eight keys per thread");
      uint64_t* lst = big_list(L);
      const uint64_t* srt = n <= 2u * kBlock   ? sort_desc_lds<2>(lst, L.big_tmp, n)
                            : n <= 4u * kBlock ? sort_desc_lds<4>(lst, L.big_tmp, n)
                                               : sort_desc_lds<8>(lst, L.big_tmp, n);
      float* buf = srt == L.big_tmp ? reinterpret_cast<float*>(big_list(L)) : reinterpret_cast<float*>(L.big_tmp);
      auto key_at = [&](uint32_t i) { return (uint32_t)(srt[i] >> 32); };
      // The tail's terms are staged by every wave.
      stage_exp_terms(buf, K, key_at, L.exptab, tid, kBlock);
      lds_barrier();
      if (wave == 0)
        draw_tail_lds<true>(a, b, len_b, P, K, key_at, [&](uint32_t i) { return ~(uint32_t)srt[i]; }, rng0, L.exptab,
                            buf);
      return true;
    }
  }
  if (n <= 128) {
    rank_in_regs<2>(L.ord, n, K, wave, lane, L.skey, L.sid);
  } else if (n <= 192) {
    rank_in_regs<3>(L.ord, n, K, wave, lane, L.skey, L.sid);
  } else if (n <= 256) {
    rank_in_regs<4>(L.ord, n, K, wave, lane, L.skey, L.sid);
  } else if (!BIGK) {
    if (n > 512u) return false;
    rank_in_regs<8>(L.ord, n, K, wave, lane, L.skey, L.sid);
  } else {
    rank_in_lds(L.ord, reinterpret_cast<uint64_t*>(L.ent), n, K, L.skey, L.sid);  // the entries are consumed
  }
  LLMHIP_MARK(10);
  lds_barrier();
  LLMHIP_MARK(7);

  // 7. The sequential tail (one wave). For K > 64 every wave stages its
  //    terms first (the candidate list's LDS is free past the rank).
  if (BIGK && K > 64u) {
    stage_exp_terms(reinterpret_cast<float*>(L.ord), K, [&](uint32_t i) { return L.skey[i]; }, L.exptab, tid, kBlock);
    lds_barrier();
  }
  if (wave == 0) {
    if (!BIGK || K <= 64u) {
      draw_tail_bcast(a, b, len_b, P, K, lane < K ? L.skey[lane] : kKeyNone, lane < K ? L.sid[lane] : 0u,
                      u_draw, st_next, L.exptab, L.tail);
    } else {
      draw_tail_lds<true>(a, b, len_b, P, K, [&](uint32_t i) { return L.skey[i]; },
                          [&](uint32_t i) { return L.sid[i]; }, rng0, L.exptab, reinterpret_cast<float*>(L.ord));
    }
  }
  LLMHIP_MARK(8);
  return true;
}

}  // namespace llmhip
