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
__device__ __forceinline__ void general_row(const SampleArgs& a, uint32_t b, GenLds& L) {
  const llmhip_params P = load_params(a, b);
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
  if (!(row_class(load_params(a, b), a.V) & a.row_class_mask)) return;
  general_row(a, b, L);
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
constexpr uint32_t kSelBits = 12;     // threshold histogram: top 12 key bits
constexpr uint32_t kSelBins = 1u << kSelBits;
constexpr uint32_t kHistWaves = 4;    // waves that load and count the history
constexpr uint32_t kHistPerThread = 4;
constexpr uint32_t kWaveCand = kFastCand / kWaves;  // per-wave candidate region

// Element e of thread t holds position ((e/4)*1024 + t)*4 + e%4: each wave
// reads 1 KiB contiguous per dwordx4 load. Position p lives in thread
// (p/4) % 1024, slot ((p/4096)*4 + p%4).
__device__ __forceinline__ uint32_t slot_pos(uint32_t e, uint32_t tid) {
  return ((e >> 2) * kBlock + tid) * 4u + (e & 3u);
}
__device__ __forceinline__ uint32_t pos_owner(uint32_t p) { return (p >> 2) & (kBlock - 1); }
__device__ __forceinline__ uint32_t pos_slot(uint32_t p) { return ((p >> 12) << 2) | (p & 3u); }

// Candidate order key: larger = earlier in the reference's sort (value desc,
// then id asc).
__device__ __forceinline__ uint64_t cand_order(uint32_t wkey, uint32_t id) {
  return ((uint64_t)wkey << 32) | (uint64_t)(0xffffffffu - id);
}

// Threshold from a 12-bit key histogram of per-thread maxima (bins zeroed
// beforehand, one atomic per thread already added): the lower edge of the
// bin holding the Q-th largest maximum, lowered by the run of keys whose
// v/T ties with it (lane l tests the key l+1 below; runs of ties are at most
// ceil(2T)+1 long, so 64 covers T < 31). Two LDS barriers; every wave
// computes the same result.
__device__ __forceinline__ uint32_t hist_threshold(const uint32_t* s_bins, uint32_t* s_seg,
                                                   uint32_t Q, float T, uint32_t wave,
                                                   uint32_t lane) {
  {
    const uint4 q = reinterpret_cast<const uint4*>(s_bins)[kSelBins / 4 - 1u - (64u * wave + lane)];
    const uint32_t tot = wave_incl_scan(q.x + q.y + q.z + q.w);
    if (lane == 63) s_seg[wave] = tot;
  }
  lds_barrier();
  const uint32_t sc = lane < kWaves ? s_seg[lane] : 0u;
  const uint32_t si = wave_incl_scan(sc);
  const uint64_t segm = __ballot(lane < kWaves && Q <= si);
  const uint32_t seg = (uint32_t)__ffsll((unsigned long long)segm) - 1u;
  const uint32_t kk = Q - (readlane_u32(si, seg) - readlane_u32(sc, seg));
  const uint4 q = reinterpret_cast<const uint4*>(s_bins)[kSelBins / 4 - 1u - (64u * seg + lane)];
  const uint32_t lt = q.x + q.y + q.z + q.w;  // descending within the lane: w, z, y, x
  const uint32_t ci = wave_incl_scan(lt);
  const uint64_t lm = __ballot(kk <= ci);
  const uint32_t l = (uint32_t)__ffsll((unsigned long long)lm) - 1u;
  const uint32_t need = kk - (readlane_u32(ci, l) - readlane_u32(lt, l));
  const uint32_t cw = readlane_u32(q.w, l), cz = readlane_u32(q.z, l), cy = readlane_u32(q.y, l);
  const uint32_t sub = need <= cw ? 0u : need <= cw + cz ? 1u : need <= cw + cz + cy ? 2u : 3u;
  const uint32_t bin = kSelBins - 1u - (4u * (64u * seg + l) + sub);
  const uint32_t tau = bin << (32 - kSelBits);
  uint32_t lo = kKeyNaN;
  if (tau > 0x007fffffu + 64u) {
    const uint32_t wt = f2key(key2f(tau) / T);
    const uint64_t ties = __ballot(f2key(key2f(tau - 1u - lane) / T) == wt);
    const uint64_t run = ~ties;
    if (run != 0ull) lo = tau - (uint32_t)(__ffsll((unsigned long long)run) - 1);
  }
  return lo > kKeyNaN ? lo : kKeyNaN;
}

// One row on the register path. Returns false (uniformly across the
// workgroup, before writing any output) when the row needs the general
// path; s_cnt is the u16 history multiplicity table (2 per word).
template <int NCH, bool VEC>
__device__ __forceinline__ bool fast_row(const SampleArgs& a, uint32_t* s_cnt) {
  __shared__ uint32_t s_pm[kBlock];      // per-thread mask of slots whose logit is penalized
  __shared__ uint32_t s_plist[kMaxPen];  // distinct penalized ids
  __shared__ __attribute__((aligned(16))) uint32_t s_bins[kSelBins];
  __shared__ uint32_t s_seg[kWaves];
  __shared__ uint32_t s_wkey[kWaves * kWaveCand];  // per-wave candidate regions: v key
  __shared__ uint32_t s_wid[kWaves * kWaveCand];   //                              id
  __shared__ __attribute__((aligned(16))) uint64_t s_ord[kFastCand];  // compacted order keys
  __shared__ uint32_t s_skey[kMaxFastK];
  __shared__ uint32_t s_sid[kMaxFastK];
  __shared__ __attribute__((aligned(16))) float s_tail[128];
  __shared__ float s_redv[kWaves];
  __shared__ uint32_t s_redi[kWaves];
  __shared__ uint32_t s_misc[8];
  static_assert(NCH * 4 <= 32, "slot mask is 32 bits");

  // The grid is exactly B workgroups.
  const uint32_t b = blockIdx.x;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const uint32_t V = a.V;
  const bool hist_wave = wave < kHistWaves;

  // 1. Loads. Waves 0-3 first fetch the history ids (their address needs
  //    the history offsets, one scalar round trip) and then their share of
  //    the row; waves 4-15 put their share of the row in flight at once.
  //    Row loads are branch-free: positions past V read position 0 and are
  //    dropped below. Parameters and RNG state are scalar loads.
  const float* row = a.logits + (size_t)b * a.ld;
  float x[NCH * 4];
  auto load_chunk = [&](int c) __attribute__((always_inline)) {
    const uint32_t base = ((uint32_t)c * kBlock + tid) * 4u;
    if (VEC) {
      const float4 q = *reinterpret_cast<const float4*>(row + (base < V ? base : 0u));
      x[4 * c + 0] = q.x;
      x[4 * c + 1] = q.y;
      x[4 * c + 2] = q.z;
      x[4 * c + 3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * c + j] = row[base + j < V ? base + j : 0u];
    }
  };
  uint32_t h0 = 0, h1 = 0;
  auto load_offsets = [&]() __attribute__((always_inline)) {
    if (a.hist_offsets && a.hist) {
      h0 = as_const(a.hist_offsets)[b];
      h1 = as_const(a.hist_offsets)[b + 1];
    }
  };
  uint32_t hid[kHistPerThread];
#pragma unroll
  for (uint32_t u = 0; u < kHistPerThread; ++u) hid[u] = 0xffffffffu;
  if (hist_wave) {
    load_offsets();
    const uint32_t H0 = h1 > h0 ? h1 - h0 : 0u;
#pragma unroll
    for (uint32_t u = 0; u < kHistPerThread; ++u) {
      const uint32_t j = tid + u * kHistWaves * 64u;
      if (j < H0) hid[u] = a.hist[h0 + j];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < NCH; ++c) load_chunk(c);
  __builtin_amdgcn_sched_barrier(0);
  if (!hist_wave) load_offsets();

  const llmhip_params P = load_params(a, b);
  const uint64_t rng0 = as_const(a.rng_state)[b];
  {
    uint4* c4 = reinterpret_cast<uint4*>(s_cnt);
    for (uint32_t i = tid; i < (V + 7) / 8; i += kBlock) c4[i] = make_uint4(0u, 0u, 0u, 0u);
    reinterpret_cast<uint4*>(s_bins)[tid] = make_uint4(0u, 0u, 0u, 0u);  // kSelBins / 4 == kBlock
    s_pm[tid] = 0u;
    if (tid < 8) s_misc[tid] = 0u;
  }
  const uint32_t cls = row_class(P, V);
  if (!(cls & a.row_class_mask)) return true;
  const float T = P.temperature, rp = P.repetition_penalty;
  const uint32_t H = (rp != 1.0f && h1 > h0) ? h1 - h0 : 0u;
  // A u16 count could overflow: take the general path.
  if (H >= 65536u) return false;
  const bool use_pen = H > 0;
  lds_barrier();

  // 2. History multiplicities (integer LDS atomics: the counts do not
  //    depend on the order), counted by waves 0-3 while the row streams in.
  //    The first occurrence of an id enlists it for one processor lane and
  //    marks its slot in the owner thread's mask.
  auto add_hist = [&](uint32_t id) __attribute__((always_inline)) {
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
  if (use_pen && hist_wave) {
#pragma unroll
    for (uint32_t u = 0; u < kHistPerThread; ++u) add_hist(hid[u]);
    for (uint32_t j = tid + kHistPerThread * kHistWaves * 64u; j < H; j += kHistWaves * 64u)
      add_hist(a.hist[h0 + j]);
  }

  // 3. Speculative threshold from the first quarter of the row (it arrives
  //    first): per-thread maxima over chunks 0..S-1 go into the key
  //    histogram while the rest of the row is still in flight. The count in
  //    6 proves or rejects it.
  constexpr int S = NCH >= 4 ? NCH / 4 : NCH;
  const uint32_t K = P.top_k;  // 0 < K < V, K <= 1024 (row class)
  const bool greedy = cls == kClassGreedy;
  auto chunk_full = [&](int c) __attribute__((always_inline)) { return (uint32_t)(c + 1) * 4u * kBlock <= V; };
  if (!greedy) {
    float sm = -INFINITY;
#pragma unroll
    for (int c = 0; c < S; ++c) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v = x[4 * c + j];
        sm = (chunk_full(c) || slot_pos(4 * c + j, tid) < V) ? fmaxf(sm, v) : sm;
      }
    }
    const uint32_t sk = slot_pos(0, tid) < V ? f2key(sm) : kKeyNone;
    atomicAdd(&s_bins[sk >> (32 - kSelBits)], 1u);
  }
  lds_barrier();
  const uint32_t D = use_pen ? s_misc[3] : 0u;
  if (D > kMaxPen) return false;

  // 4. Processor lanes: each distinct penalized id is gathered once (its
  //    line is being streamed by the row loads, so this merges in L2) and
  //    gets mask -> penalty (m times in sequence: no float atomics) here.
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
  // Logit v as the sampler sees it before temperature (mask applied) for a
  // slot this thread owns; penalized slots are handled by processor lanes.
  auto slot_ok = [&](int e) __attribute__((always_inline)) {
    const uint32_t pos = slot_pos(e, tid);
    return (chunk_full(e >> 2) || pos < V) && !((pm >> e) & 1u) && !(a.allowed && masked_out(a, pos));
  };

  if (greedy) {
    // ops/loss.rs:6-16 over the penalized, masked row (before temperature).
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) {
      const float v = x[e];
      if (v > bv && slot_ok(e)) {
        bv = v;
        bi = slot_pos(e, tid);
      }
    }
    // A masked slot is -inf, which never beats anything; a masked-out slot
    // skipped above is therefore equivalent.
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
    return true;
  }
  // 5. Speculative threshold: aim at ~1.6 K candidates over the full row.
  //    A threshold at or below -inf (fewer than K finite logits in reach)
  //    goes to the general path.
  uint32_t thr;
  {
    const uint32_t Q = S == NCH ? K : (uint32_t)((8u * K * S + 5u * NCH - 1u) / (5u * NCH)) + 2u;
    thr = hist_threshold(s_bins, s_seg, Q, T, wave, lane);
  }
  if (thr <= 0x007fffffu) return false;

  // 6. Candidates: v >= thr. Dividing by T > 0 is monotone, so the top-k by
  //    v/T lies among them once there are at least K (the threshold was
  //    lowered by the values the division merges into ties with it). The
  //    scan is one compare per logit; the rare hits go to this wave's own
  //    LDS region through a ballot, so no cross-wave offsets are needed.
  //    Each wave then turns its hits into post-temperature order keys (one
  //    division per hit, generate.rs:357-359) and appends them to the
  //    compact list with one LDS atomic.
  // Hits go to this wave's region as (raw value bits, position): one compare
  // per logit, and for the rare slots where some lane hits, a ballot offset
  // and two LDS writes. Validity (penalized slot, padding, mask) and keys
  // are settled per hit afterwards, one lane per hit.
  auto scan_own = [&](float tf, uint32_t& cnt) __attribute__((always_inline)) {
    uint32_t* rk = s_wkey + wave * kWaveCand;
    uint32_t* ri = s_wid + wave * kWaveCand;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) {
      const bool hit = x[e] >= tf;
      const uint64_t m = __ballot(hit);
      if (m) {
        const uint32_t o = cnt + lanes_below(m);
        if (hit && o < kWaveCand) {
          rk[o] = __float_as_uint(x[e]);
          ri[o] = slot_pos(e, tid) | ((uint32_t)e << 24);
        }
        cnt += (uint32_t)__popcll((unsigned long long)m);
      }
    }
  };
  // Processor values (they wait for the gathers, which complete after the
  // row): mask -> penalty m times in sequence.
  float gx[kPenPerThread];  // NaN = none
  auto finish_processors = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t r = 0; r < kPenPerThread; ++r) {
      gx[r] = __uint_as_float(0x7fc00000u);
      if (gp[r] != 0xffffffffu) {
        float v = gv[r];
        if (masked_out(a, gp[r])) v = -INFINITY;
        gx[r] = apply_penalty(v, gm[r], rp);
      }
    }
  };
  auto collect_rest = [&](float tf, uint32_t cnt, uint32_t counter) __attribute__((always_inline)) {
    uint32_t* rk = s_wkey + wave * kWaveCand;
    uint32_t* ri = s_wid + wave * kWaveCand;
#pragma unroll
    for (uint32_t r = 0; r < kPenPerThread; ++r) {
      const bool hit = gx[r] >= tf;
      const uint64_t m = __ballot(hit);
      if (m) {
        const uint32_t o = cnt + lanes_below(m);
        if (hit && o < kWaveCand) {
          rk[o] = __float_as_uint(gx[r]);
          ri[o] = gp[r] | 0xff000000u;  // processor value: always valid
        }
        cnt += (uint32_t)__popcll((unsigned long long)m);
      }
    }
    if (cnt > kWaveCand) {
      if (lane == 0) atomicOr(&s_misc[7], 1u);  // region overflow
      return;
    }
    // Settle each hit: owner slots that are penalized (their processor
    // lane stands in), padding or masked are dropped; the rest get their
    // post-temperature order key (one division per hit, generate.rs:357-359).
    for (uint32_t k = lane; k < cnt; k += 64) {
      const float v = __uint_as_float(rk[k]);
      const uint32_t w = ri[k];
      const uint32_t pos = w & 0x00ffffffu, e = w >> 24;
      bool ok = true;
      if (e != 0xffu) {
        // owner slot: the owner's penalized mask lives in LDS
        ok = pos < V && !((s_pm[pos_owner(pos)] >> e) & 1u) && !(a.allowed && masked_out(a, pos));
      }
      const uint64_t mk = __ballot(ok);
      uint32_t base = 0u;
      if (lane == 0 && mk) base = atomicAdd(&s_misc[counter], (uint32_t)__popcll((unsigned long long)mk));
      base = readlane_u32(base, 0);
      const uint32_t o = base + lanes_below(mk);
      if (ok && o < kFastCand) s_ord[o] = cand_order(f2key(v / T), pos);
    }
  };
  auto collect = [&](uint32_t th, uint32_t counter) __attribute__((always_inline)) {
    const float tf = key2f(th);
    uint32_t cnt = 0u;
    scan_own(tf, cnt);
    finish_processors();
    collect_rest(tf, cnt, counter);
  };
  collect(thr, 2);
  lds_barrier();
  uint32_t n = s_misc[2];
  if (n < K || n > kFastCand || s_misc[7]) {
    // The speculative threshold failed: use the exact one, the lower edge of
    // the bin holding the K-th largest of the 1024 per-thread maxima (at
    // least K logits lie at or above it, in the threads whose maximum
    // does). The count table is dead by now: it holds the histogram.
    uint32_t* bins2 = s_cnt;
    reinterpret_cast<uint4*>(bins2)[tid] = make_uint4(0u, 0u, 0u, 0u);
    float tm = -INFINITY;
#pragma unroll
    for (int e = 0; e < NCH * 4; ++e) tm = slot_ok(e) ? fmaxf(tm, x[e]) : tm;
#pragma unroll
    for (uint32_t r = 0; r < kPenPerThread; ++r) tm = fmaxf(tm, gx[r]);
    if (tid == 0) s_misc[7] = 0u;
    lds_barrier();
    atomicAdd(&bins2[(tm == tm ? f2key(tm) : kKeyNone) >> (32 - kSelBits)], 1u);
    lds_barrier();
    thr = hist_threshold(bins2, s_seg, K, T, wave, lane);
    if (thr <= 0x007fffffu) return false;
    collect(thr, 6);
    lds_barrier();
    n = s_misc[6];
    // Heavy ties or an unusually flat top: not bounded by the register
    // path.
    if (n > kFastCand || s_misc[7]) return false;
  }

  // 7. Ranks by (w key desc, id asc): rank(i) = #{j : ord_j > ord_i}. Each
  //    wave takes an even slice of the list; lanes hold the whole list (up
  //    to 4 keys each) and one ballot per lane-slot counts the keys that
  //    come first.
  {
    const uint32_t per = (n + kWaves - 1) / kWaves;
    const uint32_t i0 = min(n, wave * per), i1 = min(n, i0 + per);
    if (n <= 256) {
      uint64_t oj[4];
#pragma unroll
      for (uint32_t t = 0; t < 4; ++t) {
        const uint32_t j = lane + 64u * t;
        oj[t] = j < n ? s_ord[j] : 0ull;
      }
      const uint64_t mi = i0 + lane < i1 ? s_ord[i0 + lane] : 0ull;
      for (uint32_t i = 0; i < i1 - i0; ++i) {
        const uint64_t oi = readlane_u64(mi, i);
        uint32_t r = 0u;
#pragma unroll
        for (uint32_t t = 0; t < 4; ++t) r += (uint32_t)__popcll((unsigned long long)__ballot(oj[t] > oi));
        if (r < K && lane == 0) {
          s_skey[r] = (uint32_t)(oi >> 32);
          s_sid[r] = 0xffffffffu - (uint32_t)oi;
        }
      }
    } else {
      for (uint32_t i = i0; i < i1; ++i) {
        const uint64_t oi = s_ord[i];
        uint32_t r = 0u;
        for (uint32_t j0 = 0; j0 < n; j0 += 64) {
          const uint32_t j = j0 + lane;
          r += (uint32_t)__popcll((unsigned long long)__ballot(j < n && s_ord[j] > oi));
        }
        if (r < K && lane == 0) {
          s_skey[r] = (uint32_t)(oi >> 32);
          s_sid[r] = 0xffffffffu - (uint32_t)oi;
        }
      }
    }
  }
  lds_barrier();

  // 8. The sequential tail (one wave).
  if (wave == 0) {
    if (K <= 64) {
      draw_tail_small(a, b, P, K, lane < K ? s_skey[lane] : kKeyNone, lane < K ? s_sid[lane] : 0u,
                      rng0, s_tail);
    } else {
      draw_tail(a, b, P, K, [&](uint32_t i) { return s_skey[i]; }, [&](uint32_t i) { return s_sid[i]; });
    }
  }
  return true;
}

template <int NCH, bool VEC>
__global__ __launch_bounds__(kBlock) void sample_fast_kernel(SampleArgs a) {
  // u16 history multiplicities; also the general path's LDS when a row
  // falls back.
  __shared__ __attribute__((aligned(16))) uint32_t s_cnt[kMaxFastV / 2];
  static_assert(sizeof(GenLds) <= sizeof(s_cnt), "general-path LDS must fit the count table");
  if (!fast_row<NCH, VEC>(a, s_cnt)) {
    __syncthreads();
    general_row(a, blockIdx.x, *reinterpret_cast<GenLds*>(s_cnt));
  }
}

// ---------------------------------------------------------------------------
// Host-side launch.
// ---------------------------------------------------------------------------
template <int NCH>
static hipError_t launch_fast_nch(const SampleArgs& a, bool vec, hipStream_t s) {
  if (vec) {
    hipLaunchKernelGGL((sample_fast_kernel<NCH, true>), dim3(a.B), dim3(kBlock), 0, s, a);
  } else {
    hipLaunchKernelGGL((sample_fast_kernel<NCH, false>), dim3(a.B), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_fast(const SampleArgs& a, bool vec, hipStream_t s) {
  if (a.V <= 4096) return launch_fast_nch<1>(a, vec, s);
  if (a.V <= 8192) return launch_fast_nch<2>(a, vec, s);
  if (a.V <= 16384) return launch_fast_nch<4>(a, vec, s);
  return launch_fast_nch<8>(a, vec, s);
}

hipError_t launch_general(const SampleArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(sample_general_kernel, dim3(a.B), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace llmhip
