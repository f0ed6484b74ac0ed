// Shared definitions of the gfx950 sampler: the SplitMix64 step, the
// order-preserving key transform and the argument block the kernels take.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/llmhip_sampler.h"
#include "glibc_expf.h"
#include "wave_ops.h"

namespace llmhip {

// crates/llm-core/src/rng.rs:16-22 (SplitMix64, one step).
__host__ __device__ __forceinline__ uint64_t splitmix64_next(uint64_t& state) {
  state += 0x9E3779B97F4A7C15ull;
  uint64_t z = state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// crates/llm-core/src/rng.rs:31-34: top 24 bits / 2^24 (exact in binary32).
__host__ __device__ __forceinline__ float next_f32(uint64_t& state) {
  return (float)(uint32_t)(splitmix64_next(state) >> 40) * 0x1p-24f;
}

// Order-preserving map from binary32 to u32: key(a) > key(b) iff a > b as
// the reference's sort sees them (partial_cmp: -0.0 == +0.0). NaN maps to 1,
// below every number (the reference's comparator is not a total order with
// NaN; rows holding NaN are outside parity). Key 0 is reserved for "no
// element" (padding, or a logit handed to another lane).
constexpr uint32_t kKeyNone = 0u;
constexpr uint32_t kKeyNaN = 1u;
__device__ __forceinline__ uint32_t f2key(float w) {
  uint32_t u = __float_as_uint(w + 0.0f);  // -0.0 + 0.0 == +0.0
  const uint32_t flip = (uint32_t)((int32_t)u >> 31) | 0x80000000u;
  u ^= flip;
  return w == w ? u : kKeyNaN;
}
__device__ __forceinline__ float key2f(uint32_t k) {
  if (k <= kKeyNaN) return __uint_as_float(0x7fc00000u);
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// One call's worth of arguments, passed by value to every kernel.
struct SampleArgs {
  const float* logits;
  uint64_t ld;
  uint32_t V;
  uint32_t B;
  const llmhip_params* params;  // device, per row (params_stride apart), or null
  uint32_t params_stride;
  llmhip_params shared;          // used when params == null
  const uint32_t* hist;          // device, may be null
  const uint32_t* hist_offsets;  // device [B+1], may be null
  // The allowed mask (generate.rs:333-341) covers ids < allowed_len, as one
  // byte per id (allowed) or one bit per id (allowed_bits: bit id % 32 of
  // word id / 32 set = allowed); at most one of the two is set.
  const uint8_t* allowed;        // device, may be null
  const uint32_t* allowed_bits;  // device, may be null
  uint32_t allowed_len;
  // Fast path: bit e of word t is set when thread t's slot e is masked out
  // by the allowed mask (the fast kernel's layout, built by a prep kernel),
  // or all zeros when there is no mask. 1024 words, always valid.
  const uint32_t* slotmask;
  // Decode-step mode (ring_cap > 0): row b's history is the last
  // min(ring_len[b] - hist_start[b], window) tokens of the ring ring[b*ring_cap
  // .. (b+1)*ring_cap) (hist == ring, hist_offsets == null); each result is
  // appended to the ring (ring_len[b] += 1), or sets done[b] at eos_id, and
  // rows with done[b] != 0 are skipped.
  uint32_t* ring;
  uint32_t* ring_len;
  uint32_t* done;
  // Decode-step mode, nullable: hist_start[b] is the first token (as a count
  // since the start of the generation) still in row b's model cache; the
  // history never reaches before it.
  const uint32_t* hist_start;
  uint32_t ring_cap;
  uint32_t window;
  // Decode-step mode, nullable: a count table per generation. counts[b *
  // counts_words + (id >> 1)] holds the u16 multiplicity of id in half
  // (id & 1), over the ring tokens counted[2b] .. counted[2b + 1] (counted
  // since the generation's start, as ring_len counts). Each step moves that
  // range to the row's window and the kernels read the multiplicities from
  // the table instead of walking the window (see counts_plan below).
  uint32_t* counts;
  uint32_t* counted;
  uint64_t counts_words;
  // Device word of kStatus* bits, set by a kernel that hit an internal
  // limit (zero after a correct call).
  uint32_t* status;
  // Device counter of rows a kernel handed to the sorting path.
  uint32_t* handovers;
  // Spins before a wait between wavefronts gives up (kSpinLimit unless a
  // test lowers it).
  uint32_t spin_limit;
  uint32_t eos_id;
  uint64_t* rng_state;
  uint32_t* out_ids;
  float* out_probs;    // may be null
  uint32_t* out_kept;  // may be null
  uint32_t* scratch;   // general path: per-row words
  uint64_t scratch_row_words;
  uint32_t row_class_mask;  // which row classes this launch handles
  // Each row's class (log2 of its RowClass bit, two bits per row: row b in
  // bits 2(b % 16) of word b / 16; zero past B), when row_cls_on. A call
  // whose rows fall into several classes runs one launch per class (or
  // group of classes); with the table, a launch's grid holds one workgroup
  // per row of its classes (launch_row), so no workgroup is spent on the
  // other rows and the working ones are consecutive, spread over all XCDs.
  // Filled by the host (which reads the parameters anyway) for calls of at
  // most kRowClsRows rows; a larger mixed call runs B workgroups per launch
  // and each finds its row's class from the row's parameters.
  uint32_t row_cls_on;
  uint32_t row_cls[128];
  // Persistent launches (the streaming path): rows of the launch (its
  // workgroups take rows j, j + gridDim.x, ...), and the device's CUs.
  uint32_t launch_rows;
  uint32_t cus;
};
constexpr uint32_t kRowClsRows = 16u * 128u;

// Row j of a launch: j, or, with the class table, the j-th row (in row
// order) of the launch's classes. Every thread of the workgroup calls it
// (full waves); lane l of each wave reads table words 2l and 2l+1 (rows
// 32l .. 32l+31).
__device__ __forceinline__ uint32_t launch_row_at(const SampleArgs& a, uint32_t j) {
  if (!a.row_cls_on) return j;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t w0 = a.row_cls[2u * lane], w1 = a.row_cls[2u * lane + 1u];
  uint32_t m0 = 0u, m1 = 0u;  // bit 2i: field i holds one of the launch's classes
#pragma unroll
  for (uint32_t c = 0; c < 4u; ++c) {
    if (!((a.row_class_mask >> c) & 1u)) continue;  // class index c is RowClass bit 1 << c
    const uint32_t x0 = w0 ^ (c * 0x55555555u), x1 = w1 ^ (c * 0x55555555u);
    m0 |= ~(x0 | (x0 >> 1)) & 0x55555555u;
    m1 |= ~(x1 | (x1 >> 1)) & 0x55555555u;
  }
  const uint32_t n = (uint32_t)(__builtin_popcount(m0) + __builtin_popcount(m1));
  const uint32_t incl = wave_incl_scan(n);
  // The grid counts the launch's rows below B only, and the zero fields
  // past B come after them in order, so the j-th match is a row below B.
  const uint32_t L = (uint32_t)__builtin_ctzll(__ballot(incl > j));
  uint32_t r = j - (readlane_u32(incl, L) - readlane_u32(n, L));
  uint32_t m = readlane_u32(m0, L), base = 32u * L;
  const uint32_t n0 = (uint32_t)__builtin_popcount(m);
  if (r >= n0) {
    r -= n0;
    m = readlane_u32(m1, L);
    base += 16u;
  }
  for (; r; --r) m &= m - 1u;
  return base + ((uint32_t)__builtin_ctz(m) >> 1);
}

// The row workgroup blockIdx.x samples (one workgroup per row of the launch).
__device__ __forceinline__ uint32_t launch_row(const SampleArgs& a) { return launch_row_at(a, blockIdx.x); }

// Workgroups of a launch over the classes in a.row_class_mask (host side).
inline uint32_t launch_grid(const SampleArgs& a) {
  if (!a.row_cls_on) return a.B;
  uint32_t n = 0;
  for (uint32_t b = 0; b < a.B; ++b) n += (a.row_class_mask >> ((a.row_cls[b >> 4] >> ((b & 15u) * 2u)) & 3u)) & 1u;
  return n;
}

// Row b's history (`recent`, generate.rs:343-352): the CSR slice
// hist[hist_offsets[b] .. hist_offsets[b+1]), or in decode-step mode the
// last H = min(ring_len[b] - hist_start[b], window) tokens of row b's ring
// (recent_tokens reads the model cache's tokens, generate.rs:178-182, which a
// cache reset trims, :187-196; the penalty only counts occurrences, so the
// ring's order does not matter).
struct HistRow {
  const uint32_t* base;  // first id of the slice, or the row's ring
  uint32_t start;        // ring: slot of the oldest token in the window
  uint32_t cap;          // ring capacity (0 for a CSR slice)
  uint32_t H;            // ids in the history
  __device__ __forceinline__ uint32_t at(uint32_t j) const {
    uint32_t k = start + j;
    if (k >= cap && cap) k -= cap;
    return base[k];
  }
};

// Tokens of row b's ring still in its model cache (decode-step mode).
__device__ __forceinline__ uint32_t ring_avail(const SampleArgs& a, uint32_t b, uint32_t len) {
  const uint32_t s = a.hist_start ? a.hist_start[b] : 0u;
  return len > s ? len - s : 0u;
}

// v0, v1: hist_offsets[b], hist_offsets[b+1] (CSR) or ring_len[b] and the
// ring tokens still in the cache (ring).
__device__ __forceinline__ HistRow hist_row(const SampleArgs& a, uint32_t b, uint32_t v0, uint32_t v1) {
  HistRow h{a.hist, 0u, 0u, 0u};
  if (a.ring_cap) {
    h.cap = a.ring_cap;
    h.H = min(min(v0, v1), a.window);
    h.base = a.ring + (size_t)b * a.ring_cap;
    h.start = (v0 - h.H) % a.ring_cap;
  } else if (a.hist && a.hist_offsets && v1 > v0) {
    h.base = a.hist + v0;
    h.H = v1 - v0;
  }
  return h;
}

// Row b's result: the id, and in decode-step mode the ring append (or the
// end of the generation at eos_id, generate.rs:157-165). len_b is
// ring_len[b] as the row read it.
__device__ __forceinline__ void store_result(const SampleArgs& a, uint32_t b, uint32_t id, uint32_t len_b) {
  a.out_ids[b] = id;
  if (a.ring_cap) {
    if (id == a.eos_id) {
      if (a.done) a.done[b] = 1u;
    } else {
      a.ring[(size_t)b * a.ring_cap + len_b % a.ring_cap] = id;
      a.ring_len[b] = len_b + 1u;
    }
  }
}

// The count table (decode-step mode with counts): at the start of a step
// the table holds the ring tokens [cs, ce); the window is [ts, te) = [len -
// H, len). When the window only slid (cs <= ts <= ce <= te), by at most
// kCountsDelta tokens in all, the tokens leaving are still in the ring and
// the table held something (an empty range leaves its contents unknown),
// one wave applies the change: -1 for tokens [cs, ts), +1 for [ce, te), as
// device-scope integer atomics (their order does not matter). Otherwise
// (the first step, a cache reset, a skipped step) the whole workgroup
// rebuilds the row: zero, then +1 per window token. Ids >= V are not
// counted, as the penalty ignores them (generate.rs:343-352).
constexpr uint32_t kCountsDelta = 32;

struct CountsPlan {
  uint32_t cs, ce, ts, te;
  bool rebuild;
};

// cs, ce: counted[2b], counted[2b + 1] as the row read them.
__device__ __forceinline__ CountsPlan counts_plan(const SampleArgs& a, uint32_t cs, uint32_t ce, uint32_t len,
                                                  uint32_t H) {
  CountsPlan p;
  p.cs = cs;
  p.ce = ce;
  p.te = len;
  p.ts = len - H;
  // An empty range says nothing about the table's contents (a generation's
  // first step): rebuild.
  p.rebuild = !(p.cs < p.ce && p.cs <= p.ts && p.ts <= p.ce && p.ce <= p.te &&
                (p.ts - p.cs) + (p.te - p.ce) <= kCountsDelta && p.te - p.cs <= a.ring_cap);
  return p;
}

__device__ __forceinline__ uint32_t* counts_row(const SampleArgs& a, uint32_t b) {
  return a.counts + (size_t)b * a.counts_words;
}

__device__ __forceinline__ uint32_t ring_token(const SampleArgs& a, uint32_t b, uint32_t t) {
  return a.ring[(size_t)b * a.ring_cap + t % a.ring_cap];
}

// Waits until this wave's table stores and atomics have been performed in
// L2, where the atomics execute and where counts_at's device-scope loads
// read. That is all the waves of one workgroup need (they share the L2 of
// their XCD); a device-scope release fence would also write back the
// XCD's whole L2 (buffer_wbl2) once per row and step. The next launch sees
// the table through the kernel boundary's own cache maintenance.
__device__ __forceinline__ void counts_publish() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The small change, by one wave (all 64 lanes). The new range is stored.
__device__ __forceinline__ void counts_slide(const SampleArgs& a, uint32_t b, const CountsPlan& p) {
  const uint32_t lane = threadIdx.x & 63u;
  uint32_t* row = counts_row(a, b);
  const uint32_t nout = p.ts - p.cs, nin = p.te - p.ce;  // nout + nin <= kCountsDelta <= 64
  if (lane < nout) {
    const uint32_t id = ring_token(a, b, p.cs + lane);
    if (id < a.V) atomicSub(&row[id >> 1], 1u << ((id & 1u) << 4));
  } else if (lane < nout + nin) {
    const uint32_t id = ring_token(a, b, p.ce + lane - nout);
    if (id < a.V) atomicAdd(&row[id >> 1], 1u << ((id & 1u) << 4));
  }
  if (lane == 0) {
    a.counted[2 * (size_t)b] = p.ts;
    a.counted[2 * (size_t)b + 1] = p.te;
  }
}

// The rebuild, by the whole workgroup (every thread calls it); ends with a
// workgroup barrier after which the row is complete in L2. A workgroup
// barrier alone does not wait for other waves' global writes to reach L2,
// where the atomics execute: every thread publishes its writes before each
// barrier.
__device__ __forceinline__ void counts_rebuild(const SampleArgs& a, uint32_t b, const CountsPlan& p) {
  uint32_t* row = counts_row(a, b);
  const uint32_t words = (a.V + 1u) / 2u;
  for (uint32_t i = threadIdx.x; i < words; i += blockDim.x)
    __hip_atomic_store(&row[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  counts_publish();
  __syncthreads();
  for (uint32_t j = threadIdx.x; j < p.te - p.ts; j += blockDim.x) {
    const uint32_t id = ring_token(a, b, p.ts + j);
    if (id < a.V) atomicAdd(&row[id >> 1], 1u << ((id & 1u) << 4));
  }
  if (threadIdx.x == 0) {
    a.counted[2 * (size_t)b] = p.ts;
    a.counted[2 * (size_t)b + 1] = p.te;
  }
  counts_publish();
  __syncthreads();
}

// Id's multiplicity in the row's table (after the step's change is
// published: device-scope loads, past the CU's cache, read L2).
__device__ __forceinline__ uint32_t counts_at(const SampleArgs& a, uint32_t b, uint32_t id) {
  const uint32_t w = __hip_atomic_load(&counts_row(a, b)[id >> 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (w >> ((id & 1u) << 4)) & 0xffffu;
}

// The step's table change for the sorting and full-vocabulary paths (every
// thread calls it): those count the window themselves, so the table is only
// kept current for the next step. Ends with every change complete.
__device__ __forceinline__ void counts_advance_all(const SampleArgs& a, uint32_t b, uint32_t len, uint32_t H) {
  const CountsPlan p = counts_plan(a, a.counted[2 * (size_t)b], a.counted[2 * (size_t)b + 1], len, H);
  if (p.rebuild) {
    counts_rebuild(a, b, p);
  } else {
    if (threadIdx.x < 64u) {
      counts_slide(a, b, p);
      counts_publish();
    }
    __syncthreads();
  }
}

enum RowClass : uint32_t {
  kClassGreedy = 1u,  // temperature <= 0
  kClassTopK = 2u,    // 0 < top_k < V and top_k <= kMaxFastK
  kClassFull = 4u,    // top_k > kMaxFastK and < V
  kClassVocab = 8u,   // top_k == 0 or top_k >= V: the whole vocabulary is kept
};

constexpr uint32_t kStatusSyncTimeout = 1u;  // an LDS wait between waves ran out of spins
constexpr uint32_t kSpinLimit = 1u << 20;    // default spins of a wait between waves (about 0.1 s)
// Words of a context's status buffer.
constexpr uint32_t kStatusHostWord = 0;      // flags of the current host-entry call
constexpr uint32_t kStatusDeviceWord = 1;    // flags of device-entry calls since the last llmhip_ctx_status
constexpr uint32_t kStatusHandoverWord = 2;  // rows handed to the sorting path since the last llmhip_ctx_status
constexpr uint32_t kStatusTakenWord = 4;     // where llmhip_ctx_status's kernel moves the device and hand-over words
constexpr uint32_t kStatusWords = 6;

constexpr uint32_t kBlock = 1024;
constexpr uint32_t kWaves = kBlock / 64;
constexpr uint32_t kMaxFastK = 4096;     // largest top_k of the register path
constexpr uint32_t kMaxFastV = 32768;    // largest V of the register path

// Chunks per lane of the fast kernel for a vocabulary of V (V <= kMaxFastV):
// each of the 1024 threads holds NCH float4 chunks of the row.
__host__ __device__ __forceinline__ uint32_t fast_nch(uint32_t V) {
  return V <= 4096 ? 1u : V <= 8192 ? 2u : V <= 16384 ? 4u : 8u;
}

__host__ __device__ __forceinline__ uint32_t row_class(const llmhip_params& p, uint32_t V) {
  // generate.rs:354: `temperature <= 0.0` (a NaN temperature is not greedy).
  if (p.temperature <= 0.0f) return kClassGreedy;
  if (p.top_k > 0 && p.top_k < V && p.top_k <= kMaxFastK) return kClassTopK;
  if (p.top_k == 0 || p.top_k >= V) return kClassVocab;
  return kClassFull;
}

// The streaming path (top-k rows past kMaxFastV) lists about 1.2 K values
// per 32768 of the row (its threshold comes from the row's first 32768
// values) in a list of kStreamCand: it takes a row when that fits with a
// margin, and when the penalty is at least 1 (one below 1 can raise a value
// past the threshold).
constexpr uint32_t kStreamSpan = 32768;
constexpr uint32_t kStreamCand = 4096;
__host__ __device__ __forceinline__ bool stream_takes(const llmhip_params& p, uint32_t V) {
  const uint32_t parts = (V + kStreamSpan - 1u) / kStreamSpan;
  return (uint64_t)p.top_k * parts * 5u <= (uint64_t)kStreamCand * 4u && p.repetition_penalty >= 1.0f;
}

// The path a row is routed to: its class, except that a top-k row past the
// register path that the streaming path does not take goes with the
// kClassFull rows (the sorting path, which selects any K <= kSelCap).
__host__ __device__ __forceinline__ uint32_t route_class(const llmhip_params& p, uint32_t V) {
  const uint32_t c = row_class(p, V);
  return c == kClassTopK && V > kMaxFastV && !stream_takes(p, V) ? kClassFull : c;
}

// Top-k rows of the sorting path with K up to kSelCap are selected and
// sorted in LDS; larger K (and full-vocabulary rows) sort the whole row in
// HBM scratch.
constexpr uint32_t kSelCap = 4096;

// Scratch words per row, in units of Vp (V rounded up to kBlock), that a row
// may touch: greedy rows and top-k rows that select in LDS use keys and
// counts; a whole-row sort (and the full-vocabulary kernel's min-p list)
// uses all five arrays.
constexpr uint32_t kScratchSelWords = 2;
constexpr uint32_t kScratchSortWords = 5;
__host__ __device__ __forceinline__ uint32_t row_scratch_words(const llmhip_params& p, uint32_t V) {
  if (p.temperature <= 0.0f) return kScratchSelWords;
  if (p.top_k > 0 && p.top_k < V && p.top_k <= kSelCap) return kScratchSelWords;
  return kScratchSortWords;
}

}  // namespace llmhip
