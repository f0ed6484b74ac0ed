// C ABI of the gfx950 sampler (declared in include/llmhip_sampler.h):
// argument validation, the per-context device scratch, host<->device
// staging for the host entry, and the choice of kernels for a batch.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "sampler_common.h"

// Device memory of llmhip_sample_device_noalloc, for callers that cannot
// allocate: each GPU the library runs on holds its own copy of this array
// until the process ends. One call lays out, from the start: the per-row
// parameters (when params_stride != 0), the allowed mask in the register
// path's slot layout (kBlock words), and the per-row scratch of the sorting
// path. Host code never passes `scratch` itself to a kernel or a copy (in
// host code the name is a host-side stand-in, not a device address): it uses
// the address hipGetSymbolAddress returns for the current device, looked up
// once per device when the first context on that device is created.
static __device__ __align__(256) uint32_t scratch[LLMHIP_NOALLOC_SCRATCH_BYTES / sizeof(uint32_t)];

namespace llmhip {
hipError_t launch_fast(const SampleArgs& a, bool vec, bool bigk, hipStream_t s);
hipError_t launch_fast_counts(const SampleArgs& a, bool vec, bool bigk, hipStream_t s);
hipError_t launch_general(const SampleArgs& a, hipStream_t s);
hipError_t launch_vocab(const SampleArgs& a, bool plain, hipStream_t s);
hipError_t launch_slotmask(const SampleArgs& a, uint32_t* out, hipStream_t s);
hipError_t launch_seen_bits(const uint32_t* tokens, uint64_t n, uint32_t V, uint32_t* bits, hipStream_t s);
hipError_t launch_take_status(uint32_t* words, hipStream_t s);
hipError_t launch_stream(const SampleArgs& a, bool vec, bool bigk, hipStream_t s);
hipError_t launch_read_floor(const float* logits, uint64_t ld, uint32_t B, uint32_t V, int read, float* out,
                             hipStream_t s);
hipError_t launch_tied_head(const float* hidden, uint64_t ldh, const float* embed, uint64_t lde, float* logits,
                            uint64_t ldl, uint32_t B, uint32_t V, uint32_t h, hipStream_t s);
}  // namespace llmhip

using namespace llmhip;

namespace {

thread_local std::string g_last_error;

}  // namespace

namespace llmhip {
// The text llmhip_last_error returns, set by code outside this file.
void set_last_error(const std::string& what) { g_last_error = what; }
}  // namespace llmhip

namespace {

int hip_fail(hipError_t e, const char* what) {
  char buf[256];
  snprintf(buf, sizeof buf, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
  g_last_error = buf;
  return e == hipErrorOutOfMemory ? LLMHIP_ERR_OUT_OF_MEMORY : LLMHIP_ERR_HIP;
}

int arg_fail(const char* what) {
  g_last_error = what;
  return LLMHIP_ERR_INVALID_ARGUMENT;
}

#define HIP_TRY(expr)                               \
  do {                                              \
    hipError_t e_ = (expr);                         \
    if (e_ != hipSuccess) return hip_fail(e_, #expr); \
  } while (0)

// A device buffer that only grows.
struct DevBuf {
  void* ptr = nullptr;
  size_t cap = 0;
  int ensure(size_t bytes) {
    if (bytes <= cap) return LLMHIP_OK;
    if (ptr) {
      hipError_t e = hipFree(ptr);
      ptr = nullptr;
      cap = 0;
      if (e != hipSuccess) return hip_fail(e, "hipFree");
    }
    size_t want = std::max<size_t>(bytes, 256);
    hipError_t e = hipMalloc(&ptr, want);
    if (e != hipSuccess) {
      ptr = nullptr;
      return hip_fail(e, "hipMalloc");
    }
    cap = want;
    return LLMHIP_OK;
  }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    cap = 0;
  }
};

}  // namespace

struct llmhip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;  // used by the host entry
  DevBuf scratch;                // general-path per-row scratch
  DevBuf params;                 // per-row params copied from the host
  DevBuf zeros;                  // kBlock zero words: the fast path's "no mask" slot mask
  DevBuf slotmask;               // kBlock words: the allowed mask in the fast path's layout
  DevBuf status;                 // kStatusWords words: kernel flags (host / device calls) and the hand-over count
  DevBuf head_logits;            // the tied head's logits when the caller does not take them
  uint32_t spin_limit = kSpinLimit;  // bound of the kernels' waits between wavefronts
  uint32_t* noalloc = nullptr;   // this device's address of the file-scope `scratch` (null: lookup failed)
  uint32_t cus = 0;              // the device's compute units (persistent launches take one workgroup each)
  // staging of the host entry
  DevBuf logits, hist, hoff, allowed, rng, ids, probs, kept;
};

namespace {

// Device address of `scratch` on each device, looked up once per device.
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
uint32_t* g_noalloc_ptr[kMaxDevices];
std::string g_noalloc_err[kMaxDevices];

// The address of `scratch` on `device`, which must be the current device.
// The first call per device looks it up; a failed lookup is kept (with its
// message) and leaves only the no-alloc entry unusable.
uint32_t* noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  if (!g_noalloc_ptr[device] && g_noalloc_err[device].empty()) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p) {
      g_noalloc_ptr[device] = static_cast<uint32_t*>(p);
    } else {
      char buf[160];
      snprintf(buf, sizeof buf, "hipGetSymbolAddress(scratch): %s (%d)", hipGetErrorString(e), (int)e);
      g_noalloc_err[device] = buf;
    }
  }
  return g_noalloc_ptr[device];
}

struct Device {
  int prev = -1;
  bool ok = false;
  explicit Device(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    ok = hipSetDevice(dev) == hipSuccess;
  }
  ~Device() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

int validate(size_t B, size_t V, size_t ld, const float* logits, const llmhip_params* params,
             const uint32_t* hist, const uint32_t* hist_offsets, const void* allowed,
             size_t allowed_len, const uint64_t* rng_state, const uint32_t* out_ids) {
  if (B == 0) return LLMHIP_OK;
  if (!params) return arg_fail("params is null");
  if (!rng_state || !out_ids) return arg_fail("rng_state and out_ids are required");
  if (V > 0x7fffffffu) return arg_fail("V must be below 2^31");
  if (B > 0x7fffffffu) return arg_fail("B must be below 2^31");
  if (V > 0 && !logits) return arg_fail("logits is null");
  if (ld < V) return arg_fail("ld < V");
  if ((hist == nullptr) != (hist_offsets == nullptr)) return arg_fail("hist and hist_offsets go together");
  if (allowed_len > 0 && !allowed) return arg_fail("allowed is null but allowed_len > 0");
  if (allowed_len > 0xffffffffu) return arg_fail("allowed_len too large");
  return LLMHIP_OK;
}

// Enqueue the kernels for one batch whose buffers are all on the device.
// `params_host` is read on the host to choose kernels; `params_dev` is its
// device copy (null when params_stride == 0).
// Decode-step mode (ring-buffer histories); ring == null for a CSR history.
// The allowed mask: one byte per id or one bit per id (at most one is set).
struct Mask {
  const uint8_t* bytes = nullptr;
  const uint32_t* bits = nullptr;
  size_t len = 0;
};

// Device memory one call works in: the context's buffers, grown as needed
// (scratch == null), or fixed regions of the no-alloc array.
struct Workspace {
  uint32_t* scratch = nullptr;  // per-row scratch, scratch_bytes long
  size_t scratch_bytes = 0;
  uint32_t* slotmask = nullptr;  // kBlock words
};

// Scratch words per row that a call may touch (row_scratch_words over its
// rows, times Vp).
size_t call_row_words(const llmhip_params* params, size_t B, size_t params_stride, size_t V) {
  uint32_t w = kScratchSelWords;
  const size_t n = params_stride ? B : 1;
  for (size_t b = 0; b < n && w < kScratchSortWords; ++b)
    w = std::max(w, row_scratch_words(params[b * params_stride], (uint32_t)V));
  const size_t Vp = (V + kBlock - 1) / kBlock * kBlock;
  return (size_t)w * Vp;
}

struct RingArgs {
  uint32_t* ring = nullptr;
  uint32_t* ring_len = nullptr;
  uint32_t* done = nullptr;
  const uint32_t* hist_start = nullptr;
  uint32_t cap = 0;
  uint32_t window = 0;
  uint32_t* counts = nullptr;   // count table (nullable)
  uint32_t* counted = nullptr;
  uint64_t counts_words = 0;
};

int enqueue(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
            const llmhip_params* params_host, size_t params_stride, const llmhip_params* params_dev,
            const uint32_t* hist, const uint32_t* hist_offsets, const Mask& mask, uint32_t eos_id,
            uint64_t* rng_state, uint32_t* out_ids, float* out_probs, uint32_t* out_kept, hipStream_t s,
            bool host_call, const RingArgs& ring = RingArgs(), const Workspace* ws = nullptr) {
  if (V == 0) {
    // Empty logits: sample_with returns 0 without drawing (generate.rs:375-377).
    HIP_TRY(hipMemsetAsync(out_ids, 0, B * sizeof(uint32_t), s));
    if (out_kept) HIP_TRY(hipMemsetAsync(out_kept, 0, B * sizeof(uint32_t), s));
    return LLMHIP_OK;
  }
  uint32_t classes = 0;
  bool bigk = false;  // some top-k row of the register path has K > 64
  bool penalized = false;  // some row has a repetition penalty (and the call a history)
  uint32_t row_cls[128] = {};  // each row's class index (SampleArgs::row_cls), for calls of <= kRowClsRows rows
  for (size_t b = 0; b < (params_stride ? B : 1); ++b) {
    const llmhip_params& p = params_host[b * params_stride];
    const uint32_t c = route_class(p, (uint32_t)V);
    classes |= c;
    bigk = bigk || (c == kClassTopK && p.top_k > 64u);
    penalized = penalized || p.repetition_penalty != 1.0f;
    if (b < kRowClsRows) row_cls[b >> 4] |= (uint32_t)__builtin_ctz(c) << ((b & 15u) * 2u);
  }
  const bool fast_ok = V <= kMaxFastV;
  const uint32_t fast_mask = fast_ok ? (classes & (kClassGreedy | kClassTopK)) : 0u;
  // Top-k rows past the register path's V stream through the persistent
  // kernel; full-vocabulary rows take the bucketed exact-fold kernel.
  const uint32_t stream_mask = fast_ok ? 0u : (classes & kClassTopK);
  const uint32_t vocab_mask = classes & kClassVocab;
  const uint32_t general_mask = classes & ~fast_mask & ~vocab_mask & ~stream_mask;

  // The fast kernel may hand a row to the general path, so scratch is
  // always sized for the batch.
  const size_t row_words = call_row_words(params_host, B, params_stride, V);
  int st = LLMHIP_OK;
  uint32_t* scr = nullptr;
  if (ws) {
    if (B * row_words * sizeof(uint32_t) > ws->scratch_bytes) return arg_fail("workspace too small for the call");
    scr = ws->scratch;
  } else {
    if ((st = ctx->scratch.ensure(B * row_words * sizeof(uint32_t)))) return st;
    scr = static_cast<uint32_t*>(ctx->scratch.ptr);
  }

  SampleArgs a{};
  a.logits = logits;
  a.ld = ld;
  a.V = (uint32_t)V;
  a.B = (uint32_t)B;
  a.params = params_stride ? params_dev : nullptr;
  a.params_stride = (uint32_t)params_stride;
  a.shared = params_host[0];
  a.hist = ring.ring ? ring.ring : hist;
  a.hist_offsets = ring.ring ? nullptr : hist_offsets;
  a.ring = ring.ring;
  a.ring_len = ring.ring_len;
  a.done = ring.done;
  a.hist_start = ring.hist_start;
  a.ring_cap = ring.cap;
  a.window = ring.window;
  a.counts = ring.counts;
  a.counted = ring.counted;
  a.counts_words = ring.counts_words;
  a.allowed = mask.len ? mask.bytes : nullptr;
  a.allowed_bits = mask.len && !mask.bytes ? mask.bits : nullptr;
  a.allowed_len = (uint32_t)mask.len;
  a.eos_id = eos_id;
  a.rng_state = rng_state;
  a.out_ids = out_ids;
  a.out_probs = out_probs;
  a.out_kept = out_kept;
  a.slotmask = static_cast<const uint32_t*>(ctx->zeros.ptr);
  a.status = static_cast<uint32_t*>(ctx->status.ptr) + (host_call ? kStatusHostWord : kStatusDeviceWord);
  a.handovers = static_cast<uint32_t*>(ctx->status.ptr) + kStatusHandoverWord;
  a.spin_limit = ctx->spin_limit;
  a.scratch = scr;
  a.scratch_row_words = row_words;
  a.cus = ctx->cus;
  // Rows of several classes: one launch per class, and each launch's
  // workgroups skip the rows of the others before reading them.
  if (params_stride && B <= kRowClsRows && __builtin_popcount(classes) > 1) {
    a.row_cls_on = 1u;
    memcpy(a.row_cls, row_cls, sizeof row_cls);
  }

  if (out_probs) HIP_TRY(hipMemsetAsync(out_probs, 0, B * V * sizeof(float), s));
  // 128-bit row loads need 16-byte aligned rows and V % 4 == 0 (a row's
  // last float4 must not extend past its V logits).
  const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) && (ld % 4 == 0) && (V % 4 == 0);
  if (fast_mask) {
    if (a.allowed || a.allowed_bits) {
      uint32_t* sm = ws ? ws->slotmask : nullptr;
      if (!sm) {
        if ((st = ctx->slotmask.ensure(kBlock * sizeof(uint32_t)))) return st;
        sm = static_cast<uint32_t*>(ctx->slotmask.ptr);
      }
      HIP_TRY(launch_slotmask(a, sm, s));
      a.slotmask = sm;
    }
    a.row_class_mask = fast_mask;
    HIP_TRY(a.counts ? launch_fast_counts(a, vec, bigk, s) : launch_fast(a, vec, bigk, s));
  }
  if (stream_mask) {
    // A row's last float4 may pass V (the stride is a multiple of 4).
    const bool svec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) && (ld % 4 == 0);
    a.row_class_mask = stream_mask;
    HIP_TRY(launch_stream(a, svec, bigk, s));
  }
  if (vocab_mask) {
    a.row_class_mask = vocab_mask;
    const bool plain = !a.allowed && !a.allowed_bits && !a.ring && !(penalized && a.hist);
    HIP_TRY(launch_vocab(a, plain, s));
  }
  if (general_mask) {
    a.row_class_mask = general_mask;
    HIP_TRY(launch_general(a, s));
  }
  return LLMHIP_OK;
}

int copy_params(llmhip_ctx* ctx, const llmhip_params* params, size_t B, size_t params_stride,
                const llmhip_params** out_dev, hipStream_t s) {
  *out_dev = nullptr;
  if (params_stride == 0) return LLMHIP_OK;
  const size_t bytes = ((B - 1) * params_stride + 1) * sizeof(llmhip_params);
  int st = ctx->params.ensure(bytes);
  if (st) return st;
  HIP_TRY(hipMemcpyAsync(ctx->params.ptr, params, bytes, hipMemcpyHostToDevice, s));
  *out_dev = static_cast<const llmhip_params*>(ctx->params.ptr);
  return LLMHIP_OK;
}

}  // namespace

namespace {

// One decode step (llmhip_decode_step and its bit-mask twin).
int decode_step(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                const llmhip_params* params, size_t params_stride, uint32_t* ring, size_t ring_cap,
                uint32_t* ring_len, uint32_t* done, const uint32_t* hist_start, size_t window, const Mask& mask,
                const void* mask_ptr, uint32_t eos_id, uint64_t* rng_state, uint32_t* out_ids, void* stream,
                uint32_t* counts = nullptr, size_t counts_words = 0, uint32_t* counted = nullptr) {
  if (!ctx) return arg_fail("ctx is null");
  int st = validate(B, V, ld, logits, params, nullptr, nullptr, mask_ptr, mask.len, rng_state, out_ids);
  if (st || B == 0) return st;
  // A generation over an empty vocabulary has no token to append.
  if (V == 0) return arg_fail("V must be at least 1 for a decode step");
  if (!ring || !ring_len) return arg_fail("ring and ring_len are required");
  if (ring_cap == 0 || ring_cap > 0x7fffffffu) return arg_fail("ring_cap must be in 1 .. 2^31-1");
  if (window > ring_cap) return arg_fail("window must not exceed ring_cap");
  if (counts || counted) {
    if (!counts || !counted) return arg_fail("counts and counted go together");
    if (counts_words < (V + 1) / 2) return arg_fail("counts_words must be at least (V + 1) / 2");
    if (window >= 65536) return arg_fail("a count table holds windows below 65536 tokens");
  }
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const llmhip_params* pdev = nullptr;
  st = copy_params(ctx, params, B, params_stride, &pdev, s);
  if (st) return st;
  RingArgs r;
  r.ring = ring;
  r.ring_len = ring_len;
  r.done = done;
  r.hist_start = hist_start;
  r.cap = (uint32_t)ring_cap;
  r.window = (uint32_t)window;
  r.counts = counts;
  r.counted = counted;
  r.counts_words = counts_words;
  return enqueue(ctx, logits, B, V, ld, params, params_stride, pdev, nullptr, nullptr, mask, eos_id, rng_state,
                 out_ids, nullptr, nullptr, s, false, r);
}

}  // namespace

extern "C" {

int llmhip_abi_version(void) { return LLMHIP_ABI_VERSION; }

const char* llmhip_status_string(int status) {
  switch (status) {
    case LLMHIP_OK: return "ok";
    case LLMHIP_ERR_INVALID_ARGUMENT: return "invalid argument";
    case LLMHIP_ERR_NO_DEVICE: return "no HIP device";
    case LLMHIP_ERR_HIP: return "HIP runtime error";
    case LLMHIP_ERR_OUT_OF_MEMORY: return "out of device memory";
    case LLMHIP_ERR_UNSUPPORTED: return "unsupported shape";
    default: return "unknown status";
  }
}

const char* llmhip_last_error(void) { return g_last_error.c_str(); }

int llmhip_ctx_create(int device, llmhip_ctx** out_ctx) {
  if (!out_ctx) return arg_fail("out_ctx is null");
  *out_ctx = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) {
    g_last_error = "no HIP device";
    return LLMHIP_ERR_NO_DEVICE;
  }
  if (device < 0 || device >= n) {
    g_last_error = "device index out of range";
    return LLMHIP_ERR_NO_DEVICE;
  }
  Device d(device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  llmhip_ctx* ctx = new llmhip_ctx();
  ctx->device = device;
  ctx->noalloc = noalloc_scratch(device);
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
    ctx->cus = (uint32_t)cus;
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return hip_fail(e, "hipStreamCreateWithFlags");
  }
  int st = ctx->zeros.ensure(kBlock * sizeof(uint32_t));
  if (st == LLMHIP_OK) st = ctx->status.ensure(kStatusWords * sizeof(uint32_t));
  if (st == LLMHIP_OK) {
    e = hipMemset(ctx->zeros.ptr, 0, kBlock * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(ctx->status.ptr, 0, kStatusWords * sizeof(uint32_t));
    if (e != hipSuccess) st = hip_fail(e, "hipMemset");
  }
  if (st != LLMHIP_OK) {
    ctx->zeros.release();
    ctx->status.release();
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return st;
  }
  *out_ctx = ctx;
  return LLMHIP_OK;
}

int llmhip_ctx_destroy(llmhip_ctx* ctx) {
  if (!ctx) return LLMHIP_OK;
  Device d(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  (void)hipDeviceSynchronize();
  for (DevBuf* b : {&ctx->scratch, &ctx->params, &ctx->zeros, &ctx->slotmask, &ctx->status, &ctx->head_logits,
                    &ctx->logits, &ctx->hist, &ctx->hoff, &ctx->allowed, &ctx->rng, &ctx->ids, &ctx->probs, &ctx->kept})
    b->release();
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return LLMHIP_OK;
}

int llmhip_sample_device(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                         const llmhip_params* params, size_t params_stride,
                         const uint32_t* hist, const uint32_t* hist_offsets,
                         const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                         uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                         uint32_t* out_kept, void* stream) {
  if (!ctx) return arg_fail("ctx is null");
  int st = validate(B, V, ld, logits, params, hist, hist_offsets, allowed, allowed_len, rng_state,
                    out_ids);
  if (st || B == 0) return st;
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const llmhip_params* pdev = nullptr;
  st = copy_params(ctx, params, B, params_stride, &pdev, s);
  if (st) return st;
  Mask m;
  m.bytes = allowed;
  m.len = allowed_len;
  return enqueue(ctx, logits, B, V, ld, params, params_stride, pdev, hist, hist_offsets, m, eos_id, rng_state,
                 out_ids, out_probs, out_kept, s, false);
}

int llmhip_sample_device_noalloc(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                                 const llmhip_params* params, size_t params_stride,
                                 const uint32_t* hist, const uint32_t* hist_offsets,
                                 const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                                 uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                                 uint32_t* out_kept, void* stream) {
  if (!ctx) return arg_fail("ctx is null");
  int st = validate(B, V, ld, logits, params, hist, hist_offsets, allowed, allowed_len, rng_state,
                    out_ids);
  if (st || B == 0) return st;
  if (!ctx->noalloc) {
    const int dev = ctx->device;
    g_last_error = dev >= 0 && dev < kMaxDevices && !g_noalloc_err[dev].empty()
                       ? g_noalloc_err[dev]
                       : std::string("no-alloc scratch: no device address for this device");
    return LLMHIP_ERR_HIP;
  }
  // The call's layout in the array: params | slot mask | per-row scratch.
  const size_t pbytes =
      params_stride ? (((B - 1) * params_stride + 1) * sizeof(llmhip_params) + 255u) / 256u * 256u : 0u;
  const size_t mbytes = kBlock * sizeof(uint32_t);
  const size_t sbytes = V ? B * call_row_words(params, B, params_stride, V) * sizeof(uint32_t) : 0u;
  if (pbytes + mbytes + sbytes > (size_t)LLMHIP_NOALLOC_SCRATCH_BYTES) {
    char buf[200];
    snprintf(buf, sizeof buf, "no-alloc scratch: the call needs %zu bytes, the maximum is %zu",
             pbytes + mbytes + sbytes, (size_t)LLMHIP_NOALLOC_SCRATCH_BYTES);
    g_last_error = buf;
    return LLMHIP_ERR_UNSUPPORTED;
  }
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* base = reinterpret_cast<uint8_t*>(ctx->noalloc);
  const llmhip_params* pdev = nullptr;
  if (params_stride) {
    HIP_TRY(hipMemcpyAsync(base, params, ((B - 1) * params_stride + 1) * sizeof(llmhip_params),
                           hipMemcpyHostToDevice, s));
    pdev = reinterpret_cast<const llmhip_params*>(base);
  }
  Workspace ws;
  ws.slotmask = reinterpret_cast<uint32_t*>(base + pbytes);
  ws.scratch = reinterpret_cast<uint32_t*>(base + pbytes + mbytes);
  ws.scratch_bytes = (size_t)LLMHIP_NOALLOC_SCRATCH_BYTES - pbytes - mbytes;
  Mask m;
  m.bytes = allowed;
  m.len = allowed_len;
  return enqueue(ctx, logits, B, V, ld, params, params_stride, pdev, hist, hist_offsets, m, eos_id, rng_state,
                 out_ids, out_probs, out_kept, s, false, RingArgs(), &ws);
}

int llmhip_sample_tied_head_device(llmhip_ctx* ctx, const float* hidden, size_t B, size_t h, size_t ldh,
                                   const float* embed, size_t V, size_t lde, const llmhip_params* params,
                                   size_t params_stride, const uint32_t* hist, const uint32_t* hist_offsets,
                                   const uint8_t* allowed, size_t allowed_len, uint32_t eos_id, uint64_t* rng_state,
                                   uint32_t* out_ids, float* out_probs, uint32_t* out_kept, float* out_logits,
                                   void* stream) {
  if (!ctx) return arg_fail("ctx is null");
  if (B == 0) return LLMHIP_OK;
  if (h > 0x7fffffffu) return arg_fail("h must be below 2^31");
  if (V > 0 && h > 0 && (!hidden || !embed)) return arg_fail("hidden and embed are required");
  if (ldh < h || lde < h) return arg_fail("ldh and lde must be at least h");
  if (V > 0x7fffffffu || B > 0x7fffffffu) return arg_fail("B and V must be below 2^31");
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The logits: the caller's [B][V] buffer, or the context's, with rows
  // padded to a multiple of 4 floats so the sampler reads them 16 bytes at
  // a time.
  float* lg = out_logits;
  size_t ldl = V;
  if (!lg && V > 0) {
    ldl = (V + 3) / 4 * 4;
    int st = ctx->head_logits.ensure(B * ldl * sizeof(float));
    if (st) return st;
    lg = static_cast<float*>(ctx->head_logits.ptr);
  }
  int st = validate(B, V, ldl, lg, params, hist, hist_offsets, allowed, allowed_len, rng_state, out_ids);
  if (st) return st;
  if (V > 0) HIP_TRY(launch_tied_head(hidden, ldh, embed, lde, lg, ldl, (uint32_t)B, (uint32_t)V, (uint32_t)h, s));
  const llmhip_params* pdev = nullptr;
  st = copy_params(ctx, params, B, params_stride, &pdev, s);
  if (st) return st;
  Mask m;
  m.bytes = allowed;
  m.len = allowed_len;
  return enqueue(ctx, lg, B, V, ldl, params, params_stride, pdev, hist, hist_offsets, m, eos_id, rng_state, out_ids,
                 out_probs, out_kept, s, false);
}

int llmhip_sample_device_bits(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                              const llmhip_params* params, size_t params_stride,
                              const uint32_t* hist, const uint32_t* hist_offsets,
                              const uint32_t* allowed_bits, size_t allowed_len, uint32_t eos_id,
                              uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                              uint32_t* out_kept, void* stream) {
  if (!ctx) return arg_fail("ctx is null");
  int st = validate(B, V, ld, logits, params, hist, hist_offsets, allowed_bits, allowed_len, rng_state,
                    out_ids);
  if (st || B == 0) return st;
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const llmhip_params* pdev = nullptr;
  st = copy_params(ctx, params, B, params_stride, &pdev, s);
  if (st) return st;
  Mask m;
  m.bits = allowed_bits;
  m.len = allowed_len;
  return enqueue(ctx, logits, B, V, ld, params, params_stride, pdev, hist, hist_offsets, m, eos_id, rng_state,
                 out_ids, out_probs, out_kept, s, false);
}

int llmhip_seen_tokens(llmhip_ctx* ctx, const uint32_t* tokens, size_t n, size_t V, uint32_t* seen_bits,
                       void* stream) {
  if (!ctx) return arg_fail("ctx is null");
  if (V == 0) return LLMHIP_OK;
  if (V > 0x7fffffffu) return arg_fail("V must be below 2^31");
  if (!seen_bits) return arg_fail("seen_bits is null");
  if (n > 0 && !tokens) return arg_fail("tokens is null but n > 0");
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  HIP_TRY(launch_seen_bits(tokens, n, (uint32_t)V, seen_bits, static_cast<hipStream_t>(stream)));
  return LLMHIP_OK;
}

int llmhip_bench_floor(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld, int read, float* out,
                       void* stream) {
  if (!ctx) return arg_fail("ctx is null");
  if (B == 0 || B > 0x7fffffffu) return arg_fail("B must be in 1 .. 2^31-1");
  if (V == 0 || V > kMaxFastV || V % 4 != 0) return arg_fail("V must be a multiple of 4 in 4 .. 32768");
  if (ld < V || ld % 4 != 0) return arg_fail("ld must be a multiple of 4, at least V");
  if (!logits || reinterpret_cast<uintptr_t>(logits) % 16 != 0) return arg_fail("logits must be 16-byte aligned");
  if (!out) return arg_fail("out is null");
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  HIP_TRY(launch_read_floor(logits, ld, (uint32_t)B, (uint32_t)V, read, out, static_cast<hipStream_t>(stream)));
  return LLMHIP_OK;
}

int llmhip_sample_host(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                       const llmhip_params* params, size_t params_stride,
                       const uint32_t* hist, const uint32_t* hist_offsets,
                       const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                       uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                       uint32_t* out_kept) {
  if (!ctx) return arg_fail("ctx is null");
  int st = validate(B, V, ld, logits, params, hist, hist_offsets, allowed, allowed_len, rng_state,
                    out_ids);
  if (st || B == 0) return st;
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  hipStream_t s = ctx->stream;
  uint32_t* host_word = static_cast<uint32_t*>(ctx->status.ptr) + kStatusHostWord;
  // This call reports only what its own kernels flag.
  HIP_TRY(hipMemsetAsync(host_word, 0, sizeof(uint32_t), s));

  // Rows are copied densely (ld = V on the device).
  const size_t nlog = B * V;
  const size_t nhist = hist ? (size_t)hist_offsets[B] : 0;
  if (hist && hist_offsets[0] != 0) return arg_fail("hist_offsets[0] must be 0");
  for (size_t b = 0; hist && b < B; ++b)
    if (hist_offsets[b + 1] < hist_offsets[b]) return arg_fail("hist_offsets must be non-decreasing");
  if ((st = ctx->logits.ensure(nlog * sizeof(float)))) return st;
  if ((st = ctx->rng.ensure(B * sizeof(uint64_t)))) return st;
  if ((st = ctx->ids.ensure(B * sizeof(uint32_t)))) return st;
  if (out_kept && (st = ctx->kept.ensure(B * sizeof(uint32_t)))) return st;
  if (out_probs && (st = ctx->probs.ensure(nlog * sizeof(float)))) return st;
  if (hist) {
    if ((st = ctx->hist.ensure(std::max<size_t>(nhist, 1) * sizeof(uint32_t)))) return st;
    if ((st = ctx->hoff.ensure((B + 1) * sizeof(uint32_t)))) return st;
  }
  if (allowed_len && (st = ctx->allowed.ensure(allowed_len))) return st;

  float* dlog = static_cast<float*>(ctx->logits.ptr);
  if (V > 0) {
    if (ld == V) {
      HIP_TRY(hipMemcpyAsync(dlog, logits, nlog * sizeof(float), hipMemcpyHostToDevice, s));
    } else {
      HIP_TRY(hipMemcpy2DAsync(dlog, V * sizeof(float), logits, ld * sizeof(float), V * sizeof(float), B,
                               hipMemcpyHostToDevice, s));
    }
  }
  HIP_TRY(hipMemcpyAsync(ctx->rng.ptr, rng_state, B * sizeof(uint64_t), hipMemcpyHostToDevice, s));
  if (hist) {
    if (nhist) HIP_TRY(hipMemcpyAsync(ctx->hist.ptr, hist, nhist * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(ctx->hoff.ptr, hist_offsets, (B + 1) * sizeof(uint32_t), hipMemcpyHostToDevice, s));
  }
  if (allowed_len) HIP_TRY(hipMemcpyAsync(ctx->allowed.ptr, allowed, allowed_len, hipMemcpyHostToDevice, s));
  const llmhip_params* pdev = nullptr;
  if ((st = copy_params(ctx, params, B, params_stride, &pdev, s))) return st;

  Mask m;
  m.bytes = allowed_len ? static_cast<const uint8_t*>(ctx->allowed.ptr) : nullptr;
  m.len = allowed_len;
  st = enqueue(ctx, dlog, B, V, V, params, params_stride, pdev,
               hist ? static_cast<const uint32_t*>(ctx->hist.ptr) : nullptr,
               hist ? static_cast<const uint32_t*>(ctx->hoff.ptr) : nullptr, m,
               eos_id, static_cast<uint64_t*>(ctx->rng.ptr), static_cast<uint32_t*>(ctx->ids.ptr),
               out_probs ? static_cast<float*>(ctx->probs.ptr) : nullptr,
               out_kept ? static_cast<uint32_t*>(ctx->kept.ptr) : nullptr, s, true);
  if (st) {
    (void)hipStreamSynchronize(s);
    return st;
  }
  HIP_TRY(hipMemcpyAsync(out_ids, ctx->ids.ptr, B * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(rng_state, ctx->rng.ptr, B * sizeof(uint64_t), hipMemcpyDeviceToHost, s));
  if (out_kept) HIP_TRY(hipMemcpyAsync(out_kept, ctx->kept.ptr, B * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  if (out_probs) HIP_TRY(hipMemcpyAsync(out_probs, ctx->probs.ptr, nlog * sizeof(float), hipMemcpyDeviceToHost, s));
  uint32_t kstatus = 0;
  HIP_TRY(hipMemcpyAsync(&kstatus, host_word, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (kstatus) {
    // A kernel hit an internal limit: its results are not trustworthy.
    g_last_error = "internal error: a workgroup sync wait timed out in the sampler kernel";
    return LLMHIP_ERR_HIP;
  }
  return LLMHIP_OK;
}

int llmhip_decode_step(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                       const llmhip_params* params, size_t params_stride, uint32_t* ring, size_t ring_cap,
                       uint32_t* ring_len, uint32_t* done, const uint32_t* hist_start, size_t window,
                       const uint8_t* allowed, size_t allowed_len, uint32_t eos_id, uint64_t* rng_state,
                       uint32_t* out_ids, void* stream) {
  Mask m;
  m.bytes = allowed;
  m.len = allowed_len;
  return decode_step(ctx, logits, B, V, ld, params, params_stride, ring, ring_cap, ring_len, done, hist_start,
                     window, m, allowed, eos_id, rng_state, out_ids, stream);
}

int llmhip_decode_step_bits(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                            const llmhip_params* params, size_t params_stride, uint32_t* ring, size_t ring_cap,
                            uint32_t* ring_len, uint32_t* done, const uint32_t* hist_start, size_t window,
                            const uint32_t* allowed_bits, size_t allowed_len, uint32_t eos_id,
                            uint64_t* rng_state, uint32_t* out_ids, void* stream) {
  Mask m;
  m.bits = allowed_bits;
  m.len = allowed_len;
  return decode_step(ctx, logits, B, V, ld, params, params_stride, ring, ring_cap, ring_len, done, hist_start,
                     window, m, allowed_bits, eos_id, rng_state, out_ids, stream);
}

int llmhip_decode_step_counts(llmhip_ctx* ctx, const float* logits, size_t B, size_t V, size_t ld,
                              const llmhip_params* params, size_t params_stride, uint32_t* ring, size_t ring_cap,
                              uint32_t* ring_len, uint32_t* done, const uint32_t* hist_start, size_t window,
                              uint32_t* counts, size_t counts_words, uint32_t* counted, const uint8_t* allowed,
                              size_t allowed_len, uint32_t eos_id, uint64_t* rng_state, uint32_t* out_ids,
                              void* stream) {
  if (!counts || !counted) return arg_fail("counts and counted are required");
  Mask m;
  m.bytes = allowed;
  m.len = allowed_len;
  return decode_step(ctx, logits, B, V, ld, params, params_stride, ring, ring_cap, ring_len, done, hist_start,
                     window, m, allowed, eos_id, rng_state, out_ids, stream, counts, counts_words, counted);
}

int llmhip_ctx_status(llmhip_ctx* ctx, void* stream, llmhip_status* out) {
  if (!ctx) return arg_fail("ctx is null");
  if (!out) return arg_fail("out is null");
  Device d(ctx->device);
  if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Read and clear in one step on the device (atomic exchanges), then copy
  // what was taken. The host entry's word stays: each host call clears it.
  uint32_t* dev = static_cast<uint32_t*>(ctx->status.ptr);
  uint32_t w[2] = {0u, 0u};
  HIP_TRY(launch_take_status(dev, s));
  HIP_TRY(hipMemcpyAsync(w, dev + kStatusTakenWord, sizeof w, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  out->flags = w[0];
  out->handovers = w[1];
  return LLMHIP_OK;
}

int llmhip_ctx_debug(llmhip_ctx* ctx, int what, uint32_t value) {
  if (!ctx) return arg_fail("ctx is null");
  switch (what) {
    case LLMHIP_DEBUG_SPIN_LIMIT:
      ctx->spin_limit = value ? value : kSpinLimit;
      return LLMHIP_OK;
    case LLMHIP_DEBUG_SET_FLAGS: {
      Device d(ctx->device);
      if (!d.ok) return hip_fail(hipErrorInvalidDevice, "hipSetDevice");
      uint32_t w = 0u;
      uint32_t* dev = static_cast<uint32_t*>(ctx->status.ptr) + kStatusDeviceWord;
      HIP_TRY(hipMemcpy(&w, dev, sizeof w, hipMemcpyDeviceToHost));
      w |= value;
      HIP_TRY(hipMemcpy(dev, &w, sizeof w, hipMemcpyHostToDevice));
      return LLMHIP_OK;
    }
    default:
      return arg_fail("unknown debug request");
  }
}

}  // extern "C"
