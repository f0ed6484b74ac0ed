/*
 * llmhip_sampler.h — C ABI of the MI355X (gfx950) decode-time sampler.
 *
 * Drop-in for scriptonait's CPU sampler:
 *   pub fn sample_with(logits: &[f32], sampling: &SamplingConfig,
 *                      recent: &[u32], rng: &mut Rng) -> u32
 *   (crates/llm-core/src/generate.rs:325-420)
 * batched over B rows. Per row it computes exactly what that function
 * computes: allowed-mask -> repetition penalty over the history -> greedy
 * exit -> temperature -> sort (value desc, id asc) -> top-k -> softmax over
 * the top-k set -> min-p -> top-p -> seeded inverse-CDF draw, and returns
 * the same token id. The reference has no FFI of its own (it is a plain
 * Rust function); a Rust host binds these symbols through the `extern "C"`
 * block shown in the integration notes, and falls back to `sample_with`
 * when a call returns non-zero, as the WebGPU path falls back to the CPU
 * (crates/wasm-app/src/inference.rs:204-214).
 *
 * Conventions
 *   - Plain pointers and sizes only. The caller owns every buffer; the
 *     library never frees caller memory.
 *   - Every entry point returns an int status: LLMHIP_OK (0) or a negative
 *     LLMHIP_ERR_* code. Nothing aborts. A degenerate row (all -inf after
 *     masking, non-finite softmax sum) is not an error: it returns the
 *     reference's fallback id, as sample_with does.
 *   - RNG: rng_state[b] is the SplitMix64 state of row b
 *     (crates/llm-core/src/rng.rs:6-22, `Rng::seed_from_u64(seed)` sets it to
 *     `seed`). It is advanced by exactly one step for every row that draws
 *     and left untouched for greedy and degenerate rows, as `Rng` is.
 *   - Not thread-safe per context: one context per host thread. Calls on
 *     one context are serialized on the stream they are given.
 */
#ifndef LLMHIP_SAMPLER_H
#define LLMHIP_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLMHIP_ABI_VERSION 7

enum {
  LLMHIP_OK = 0,
  LLMHIP_ERR_INVALID_ARGUMENT = -1, /* null pointer, ld < V, bad sizes */
  LLMHIP_ERR_NO_DEVICE = -2,        /* no HIP device / device index out of range */
  LLMHIP_ERR_HIP = -3,              /* a HIP runtime call failed (see llmhip_last_error) */
  LLMHIP_ERR_OUT_OF_MEMORY = -4,    /* device scratch could not be allocated */
  LLMHIP_ERR_UNSUPPORTED = -5       /* shape outside what this build handles */
};

/*
 * Per-row sampling parameters: the numeric fields of SamplingConfig
 * (crates/llm-core/src/generate.rs:25-80). `repetition_window` stays with
 * the caller (it decides how much history to pass, generate.rs:178-182),
 * `seed` is the initial rng_state, and `allowed` is passed separately.
 */
typedef struct llmhip_params {
  float temperature;        /* <= 0 means greedy (argmax, no draw) */
  uint32_t top_k;           /* 0 disables */
  float top_p;              /* >= 1 disables */
  float min_p;              /* <= 0 disables */
  float repetition_penalty; /* == 1 disables (history is then not read) */
} llmhip_params;

typedef struct llmhip_ctx llmhip_ctx;

/* Library ABI version (LLMHIP_ABI_VERSION of the build). No reference
 * counterpart. */
int llmhip_abi_version(void);

/* Human-readable text for a status code. No reference counterpart. */
const char* llmhip_status_string(int status);

/* Text of the last HIP error seen on this thread, or "". */
const char* llmhip_last_error(void);

/* Create a context bound to HIP device `device`. The context owns the
 * device scratch reused across calls (the reference allocates a Vec per
 * call, generate.rs:331 and :364; here nothing is allocated in steady
 * state). */
int llmhip_ctx_create(int device, llmhip_ctx** out_ctx);

/* Destroy a context and release its scratch. Null is accepted. */
int llmhip_ctx_destroy(llmhip_ctx* ctx);

/*
 * Batched sample_with on HOST buffers (replaces generate.rs:325-420 at its
 * call sites generate.rs:159 and crates/wasm-app/src/inference.rs:327).
 * Copies the inputs to the device, runs the kernels, copies the results
 * back and synchronizes before returning, so results are visible like the
 * reference's return value.
 *
 *   logits        [B][ld] f32, row b's V logits start at logits + b*ld (ld >= V)
 *   params        one llmhip_params per row, params[b * params_stride];
 *                 params_stride == 0 shares params[0] across all rows
 *   hist          concatenated token histories (`recent`), u32 ids; ids >= V
 *                 are ignored, as work.get_mut(id) ignores them
 *   hist_offsets  [B+1] CSR offsets: row b's history is
 *                 hist[hist_offsets[b] .. hist_offsets[b+1]); both may be
 *                 null for "no history"
 *   allowed       nullable [allowed_len] u8 mask shared by all rows
 *                 (SamplingConfig::allowed); ids >= allowed_len and eos_id
 *                 are always allowed
 *   eos_id        the end-of-text id (tokenizer::EOS = 258,
 *                 crates/llm-core/src/tokenizer.rs:38)
 *   rng_state     [B] u64 in/out
 *   out_ids       [B] u32 sampled ids
 *   out_probs     nullable [B][V] f32: post-truncation probabilities
 *                 scattered by id (the `probs` the draw walks over,
 *                 normalized over the top-k set), zero elsewhere; debug
 *                 output, costs an extra B*V*4 bytes of writes
 *   out_kept      nullable [B] u32: number of candidates the draw walked
 *                 over (0 for greedy and degenerate rows)
 */
int llmhip_sample_host(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                       const llmhip_params* params, size_t params_stride,
                       const uint32_t* hist, const uint32_t* hist_offsets,
                       const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                       uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                       uint32_t* out_kept);

/*
 * The same computation on DEVICE buffers (every pointer except `params`,
 * which stays on the host and is copied, is a device pointer; same meaning
 * as above), stream-ordered on `stream` (a
 * hipStream_t; null = the default stream). Returns after enqueueing; the
 * results are ready when the stream reaches that point. For decode loops
 * whose logits, history and RNG state already live in HBM: nothing crosses
 * PCIe. Scratch comes from the context (grown on first use of a larger
 * shape, which is the only time this call allocates).
 */
int llmhip_sample_device(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                         const llmhip_params* params, size_t params_stride,
                         const uint32_t* hist, const uint32_t* hist_offsets,
                         const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                         uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                         uint32_t* out_kept, void* stream);

/*
 * llmhip_sample_device for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference: its sampler allocates a Vec per call (generate.rs:331,
 * :364). Same arguments, meaning and results as
 * llmhip_sample_device; the difference is where the device memory comes
 * from. This call allocates nothing: the per-row parameters (params_stride
 * != 0), the allowed mask's slot layout and the sorting path's per-row
 * scratch go into one array of LLMHIP_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU it runs on, until the process ends. A call needs
 *   ceil(((B - 1) * params_stride + 1) * 20 / 256) * 256   (params, if per row)
 *   + 4096                                                 (mask layout)
 *   + B * w * Vp * 4                                       (scratch)
 * bytes, with Vp = V rounded up to 1024 and w = 2 when every row is greedy
 * or has 0 < top_k <= 4096, top_k < V, else 5. A larger call returns
 * LLMHIP_ERR_UNSUPPORTED (llmhip_last_error gives both sizes) and enqueues
 * nothing. The B = 256, V = 32000 top-k batch needs 64 MiB.
 * Every call on one GPU shares that GPU's array, whichever context makes it:
 * calls that overlap on one GPU (on different streams, or from different
 * threads) race and must be serialized by the caller. The kernels write
 * every scratch word they read within the call, so the array's contents
 * from an earlier call do not matter.
 * The call is not meant for recording into a HIP graph: it reads params on
 * the host to choose the kernels (a replay would keep the choice made at
 * capture), copies per-row params from the caller's host memory with
 * hipMemcpyAsync, and clears out_probs (when given) with hipMemsetAsync.
 */
#define LLMHIP_NOALLOC_SCRATCH_BYTES (96u << 20)
int llmhip_sample_device_noalloc(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                                 const llmhip_params* params, size_t params_stride,
                                 const uint32_t* hist, const uint32_t* hist_offsets,
                                 const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                                 uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                                 uint32_t* out_kept, void* stream);

/*
 * The tied output head and the sampler in one call, on device buffers:
 * logits = hidden @ embed^T (crates/llm-core/src/model.rs:396-397,
 * ops::linear_fwd(&final_normed, &weights.embed, 1, h, vocab), batched over
 * B rows), then llmhip_sample_device on those logits. Every logit is the
 * reference's dot product bit for bit (crates/llm-core/src/ops/linear.rs:
 * 19-32: four accumulators over the chunks of 4, binary32 products and
 * adds with no fused multiply-add, ((acc0 + acc1) + (acc2 + acc3)) + the
 * remainder's fold), so the ids are those of sample_with on the CPU
 * model's logits. Replaces the per-token logits read-back of
 * crates/llm-gpu/src/model.rs:481-490.
 *
 *   hidden      device [B][ldh] f32: the final-normed hidden rows
 *               (`final_normed`, one per generation)
 *   embed       device [V][lde] f32: the embedding table, tied with the head
 *   out_logits  nullable device [B][V] f32: receives the logits; null keeps
 *               them in the context (they are consumed by the sampler)
 * Every other argument is llmhip_sample_device's. Stream-ordered.
 */
int llmhip_sample_tied_head_device(llmhip_ctx* ctx, const float* hidden, size_t B, size_t h, size_t ldh,
                                   const float* embed, size_t V, size_t lde, const llmhip_params* params,
                                   size_t params_stride, const uint32_t* hist, const uint32_t* hist_offsets,
                                   const uint8_t* allowed, size_t allowed_len, uint32_t eos_id, uint64_t* rng_state,
                                   uint32_t* out_ids, float* out_probs, uint32_t* out_kept, float* out_logits,
                                   void* stream);

/*
 * One decode step for B generations whose state lives in HBM
 * (Generator::step with recent_tokens, crates/llm-core/src/generate.rs:
 * 157-165 and 178-182). For every row b with done[b] == 0 it samples from
 * the row's logits exactly as llmhip_sample_device does, with `recent` =
 * the last min(ring_len[b] - hist_start[b], window) tokens of the row's
 * history, then
 *   - at eos_id: sets done[b] = 1 (Generator::step returns None), and
 *   - otherwise: appends the token, ring[b*ring_cap + ring_len[b] %
 *     ring_cap] = id, ring_len[b] += 1 (Generator::advance).
 * Rows with done[b] != 0 are skipped: out_ids[b] = eos_id, no draw. The
 * model's forward pass for the appended token is the caller's. Nothing
 * crosses PCIe; stream-ordered on `stream` like llmhip_sample_device.
 *
 *   ring      device [B][ring_cap] u32: row b's token history (prompt and
 *             generated tokens) as a ring; the caller fills it with the
 *             prompt and sets ring_len. The prompt is what Generator::new
 *             prefills (generate.rs:131-139): an empty prompt is [BOS], and
 *             a prompt longer than context_len keeps only its last
 *             context_len tokens; the caller applies both rules before it
 *             fills the ring, so that step 1's `recent` is the reference's
 *   ring_len  device [B] u32 in/out: tokens row b has seen so far
 *   done      device nullable [B] u32 in/out
 *   hist_start device nullable [B] u32: the first token (counted from the
 *             start of row b's history, as ring_len counts) still in the
 *             row's model cache. recent_tokens reads the cache's tokens
 *             (generate.rs:178-182), and a cache reset keeps only the last
 *             context_len / 2 of them (maybe_reset_cache, generate.rs:
 *             187-196): a caller whose window can exceed what a reset keeps
 *             sets hist_start[b] = ring_len[b] - keep when it resets row b's
 *             cache (before it appends the token that follows). Null: the
 *             whole ring is in the cache.
 *   window    repetition_window (SamplingConfig, generate.rs:25-80), at
 *             most ring_cap
 * params is a host pointer, as in llmhip_sample_device; logits, allowed,
 * rng_state and out_ids are device pointers. V must be at least 1.
 */
int llmhip_decode_step(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                       const llmhip_params* params, size_t params_stride, uint32_t* ring, size_t ring_cap,
                       uint32_t* ring_len, uint32_t* done, const uint32_t* hist_start, size_t window,
                       const uint8_t* allowed, size_t allowed_len, uint32_t eos_id, uint64_t* rng_state,
                       uint32_t* out_ids, void* stream);

/*
 * llmhip_decode_step with incremental history counts, for long repetition
 * windows. The generation's `recent` multiplicities (generate.rs:343-352
 * counts each occurrence) are kept in a count table in HBM and moved with
 * the window at every step instead of being recounted from the window's
 * tokens: tokens that leave the window are subtracted and tokens that
 * enter are added (device-scope integer atomics), and the top-k path reads
 * the multiplicities only at its candidate ids. A first step, a cache
 * reset (hist_start moved) or any jump of more than 32 tokens rebuilds the
 * row's table from the ring. Results are llmhip_decode_step's.
 *
 *   counts        device [B][counts_words] u32: id's u16 multiplicity in
 *                 half (id & 1) of word id >> 1; counts_words >= (V+1)/2.
 *                 An empty range (the caller zero-fills counted at a
 *                 generation's start) leaves the table's contents unknown:
 *                 the next step rebuilds the row whatever it holds.
 *   counted       device [B][2] u32 in/out: the ring tokens (counted from
 *                 the generation's start) the table holds, [counted[2b],
 *                 counted[2b+1])
 * window must be below 65536; ring_cap must hold the window plus the
 * tokens a step adds (it does when ring_cap > window). Every other argument
 * is llmhip_decode_step's. Measured per step on B = 256, V = 32000 with
 * config 3's parameters, windows filling with generated tokens: 13.4,
 * 14.1 and 16.4 us at windows of 1024, 4096 and 16384 tokens, against
 * 13.0, 14.6 and 21.5 us for llmhip_decode_step, which recounts the
 * window: the table pays from a few thousand tokens on.
 */
int llmhip_decode_step_counts(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                              const llmhip_params* params, size_t params_stride, uint32_t* ring, size_t ring_cap,
                              uint32_t* ring_len, uint32_t* done, const uint32_t* hist_start, size_t window,
                              uint32_t* counts, size_t counts_words, uint32_t* counted, const uint8_t* allowed,
                              size_t allowed_len, uint32_t eos_id, uint64_t* rng_state, uint32_t* out_ids,
                              void* stream);

/*
 * The allowed mask as bits, built on the device from a corpus's tokens
 * (replaces Corpus::seen_tokens, crates/llm-core/src/corpus.rs:236-247,
 * which generation passes as SamplingConfig::allowed on every call,
 * crates/wasm-app/src/inference.rs:170). Bit id % 32 of word id / 32 of
 * seen_bits is set when some tokens[i] == id; ids >= V are ignored, as
 * seen.get_mut(id) ignores them. seen_bits has ceil(V / 32) words and is
 * overwritten (the bits past V are cleared). tokens and seen_bits are
 * device pointers; stream-ordered on `stream`. A corpus concatenates its
 * sources' token lists into `tokens`; their order does not matter.
 */
int llmhip_seen_tokens(llmhip_ctx* ctx, const uint32_t* tokens, size_t n, size_t V, uint32_t* seen_bits,
                       void* stream);

/*
 * llmhip_sample_device with the allowed mask as bits (as llmhip_seen_tokens
 * writes them) instead of one byte per id: id < allowed_len is masked out
 * when its bit is clear and id != eos_id (generate.rs:333-341, the same
 * rule as the byte mask). A decode loop builds the mask once per
 * generation and reads V / 8 bytes of it per call instead of V.
 */
int llmhip_sample_device_bits(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                              const llmhip_params* params, size_t params_stride,
                              const uint32_t* hist, const uint32_t* hist_offsets,
                              const uint32_t* allowed_bits, size_t allowed_len, uint32_t eos_id,
                              uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                              uint32_t* out_kept, void* stream);

/* llmhip_decode_step with the allowed mask as bits (see above). */
int llmhip_decode_step_bits(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                            const llmhip_params* params, size_t params_stride, uint32_t* ring, size_t ring_cap,
                            uint32_t* ring_len, uint32_t* done, const uint32_t* hist_start, size_t window,
                            const uint32_t* allowed_bits, size_t allowed_len, uint32_t eos_id,
                            uint64_t* rng_state, uint32_t* out_ids, void* stream);

/*
 * Status of a context's stream-ordered calls (no reference counterpart: the
 * reference's sampler cannot fail). The device entries above return once
 * their kernels are enqueued, so a kernel that hits an internal limit (a
 * wait between wavefronts that ran out of spins; a bug, never an input
 * condition) records it in a device word instead. This call waits for
 * `stream`, reads the words that the device entries' kernels set since the
 * last call, and clears them, each in one atomic exchange on the device (a
 * flag that a kernel on another stream sets meanwhile is reported now or by
 * the next call, never lost). llmhip_sample_host keeps a word of its own,
 * cleared at its start, and reports its own kernels' flags as its return
 * status.
 *   flags      LLMHIP_KSTATUS_* bits of device-entry calls (0: all well; the
 *              ids of a flagged call are not trustworthy)
 *   handovers  rows that the register or the full-vocabulary kernel handed
 *              to the sorting path, in calls of any entry (a performance
 *              figure: the ids are the reference's either way)
 */
#define LLMHIP_KSTATUS_SYNC_TIMEOUT 1u
typedef struct llmhip_status {
  uint32_t flags;
  uint32_t handovers;
} llmhip_status;
int llmhip_ctx_status(llmhip_ctx* ctx, void* stream, llmhip_status* out);

/*
 * Reader of scriptonait's checkpoint files ("SCCK", crates/llm-core/src/
 * checkpoint.rs:11-24), so a real model's embedding table can feed
 * llmhip_sample_tied_head_device. Host-side, no device work.
 *
 * llmhip_scck_parse checks `bytes` as Checkpoint::from_bytes does
 * (checkpoint.rs:192-262: magic, version 2 to 4, ModelConfig::validate, the
 * weight dtype, the tokenizer blob, the vocabulary-size consistency check,
 * the weight length) and fills `out`. Fields a version lacks read as the
 * reference's "not set" defaults (tokens_seen 0 before v3; planned_steps 0
 * and plateau_scale 1.0 before v4). A file the reference rejects returns
 * LLMHIP_ERR_INVALID_ARGUMENT, with the reason in llmhip_last_error.
 *
 * llmhip_scck_read_params widens `count` parameters, starting at parameter
 * `first` in ModelWeights::tensors() order (model.rs:75-82: embed
 * [vocab_size][hidden_dim] is parameters 0 .. vocab_size * hidden_dim,
 * final_norm_gain the last hidden_dim), to f32 in `out` (host memory). bf16
 * files widen as from_bf16 does (crates/llm-core/src/bf16.rs:22-25).
 */
typedef struct llmhip_scck_info {
  uint32_t version;
  uint32_t num_layers, hidden_dim, num_heads, num_kv_heads, context_len, local_window, vocab_size;
  float rope_theta;
  uint32_t use_ple;
  uint64_t step;
  uint64_t tokens_seen;
  uint32_t planned_steps;
  float plateau_scale;
  uint32_t weight_dtype; /* 0 = f32, 1 = bf16 */
  uint32_t num_merges;   /* the tokenizer's merges: vocab_size = 264 + num_merges */
  uint64_t tokenizer_offset, tokenizer_bytes;
  uint64_t weights_offset, weights_bytes;
  uint64_t param_count;
} llmhip_scck_info;
int llmhip_scck_parse(const uint8_t* bytes, size_t len, llmhip_scck_info* out);
int llmhip_scck_read_params(const uint8_t* bytes, size_t len, const llmhip_scck_info* info, uint64_t first,
                            uint64_t count, float* out);

/*
 * Benchmark helper (no reference counterpart): the floors the register-path
 * kernel is measured against. One launch on `stream` of B workgroups of 1024
 * threads, the sampling kernel's grid for V <= 32768. With read != 0 each
 * workgroup loads row b of `logits` (V floats, row stride ld) exactly as the
 * sampling kernel does (each lane its 16-byte chunks, nontemporal, issued
 * back to back) and does nothing else: the streaming-read floor of that
 * access shape. With read == 0 it loads nothing: the dispatch floor. out[B]
 * is written only for a NaN sum no finite row has (it keeps the loads).
 * V must be a multiple of 4 up to 32768, ld a multiple of 4 (>= V), and
 * logits 16-byte aligned; otherwise LLMHIP_ERR_INVALID_ARGUMENT.
 */
int llmhip_bench_floor(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld, int read, float* out,
                       void* stream);

/*
 * Test hooks (no reference counterpart), to exercise the error paths
 * without a kernel fault or hang:
 *   LLMHIP_DEBUG_SPIN_LIMIT  later calls on ctx bound each wait between
 *                            wavefronts by `value` spins (0: the default,
 *                            about 0.1 s); a wait that runs out flags
 *                            LLMHIP_KSTATUS_SYNC_TIMEOUT and the kernel
 *                            still finishes
 *   LLMHIP_DEBUG_SET_FLAGS   ORs `value` into the device-entry flags
 */
#define LLMHIP_DEBUG_SPIN_LIMIT 1
#define LLMHIP_DEBUG_SET_FLAGS 2
int llmhip_ctx_debug(llmhip_ctx* ctx, int what, uint32_t value);

#ifdef __cplusplus
}
#endif

#endif /* LLMHIP_SAMPLER_H */
