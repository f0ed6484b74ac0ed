// Reader of scriptonait's single-file checkpoints ("SCCK"), host code.
//
// crates/llm-core/src/checkpoint.rs:11-24 (format), :192-262
// (Checkpoint::from_bytes): a little-endian header (magic, version, seven
// u32 shape fields, rope_theta, use_ple, step, tokens_seen (v3+),
// planned_steps and plateau_scale (v4+), the weight dtype), the tokenizer
// as a length-prefixed blob (tokenizer.rs:348-390, "SCTK" v1: merge pairs),
// and the weights as a length-prefixed blob of every parameter in the
// order of ModelWeights::tensors() (model.rs:75-82: embed [vocab][hidden]
// first, then each layer's tensors, then final_norm_gain), f32 or bf16
// (the top 16 bits of each f32, bf16.rs:22-25).
//
// The reader accepts exactly the files from_bytes accepts, checking in the
// same order: ModelConfig::validate
// (config.rs:169-217, with its parameter and activation-memory estimates,
// config.rs:245-300, 346-355), the tokenizer's own checks, the
// vocabulary-size consistency check and the weight length. It does not
// build the model: parameters are widened to f32 on request, by range, so
// a caller can take the tied head's embedding table (the first
// vocab * hidden parameters) without holding the rest.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/llmhip_sampler.h"

namespace llmhip {
void set_last_error(const std::string& what);
}

namespace {

constexpr uint32_t kVersion = 4, kMinVersion = 2;  // checkpoint.rs:57-58
constexpr uint32_t kFirstMergeId = 264;           // tokenizer.rs:49 (BASE_VOCAB_SIZE)
constexpr uint64_t kMaxTrainingBytes = 2ull * 1024 * 1024 * 1024;  // config.rs:163

struct Reader {
  const uint8_t* bytes;
  size_t len, at;
  bool take(size_t n, const uint8_t** out, std::string& err) {
    if (n > len || at > len - n) {
      char buf[160];
      snprintf(buf, sizeof buf, "checkpoint truncated: wanted %zu bytes at offset %zu, file is %zu bytes", n, at, len);
      err = buf;
      return false;
    }
    *out = bytes + at;
    at += n;
    return true;
  }
  bool u32(uint32_t* v, std::string& err) {
    const uint8_t* p;
    if (!take(4, &p, err)) return false;
    memcpy(v, p, 4);
    return true;
  }
  bool u64(uint64_t* v, std::string& err) {
    const uint8_t* p;
    if (!take(8, &p, err)) return false;
    memcpy(v, p, 8);
    return true;
  }
  bool f32(float* v, std::string& err) {
    const uint8_t* p;
    if (!take(4, &p, err)) return false;
    memcpy(v, p, 4);
    return true;
  }
};

// config.rs:149-153
uint64_t ffn_dim(uint64_t hidden) { return ((hidden * 8) / 3 + 31) / 32 * 32; }

// Sizes in 128 bits: a header's u32 fields can make the 64-bit products
// wrap, and a wrapped size must not pass the memory check.
typedef unsigned __int128 u128;

// config.rs:245-264
u128 param_count(const llmhip_scck_info& c) {
  const u128 v = c.vocab_size, h = c.hidden_dim, f = ffn_dim(c.hidden_dim);
  const u128 kv = (u128)c.num_kv_heads * (c.hidden_dim / c.num_heads);
  const u128 ple = c.use_ple ? v * h : 0;
  const u128 attn = h + 2 * h * h + 2 * kv * h;
  const u128 mlp = h + 3 * h * f;
  return v * h + (u128)c.num_layers * (ple + attn + mlp) + h;
}

// config.rs:281-300
u128 activation_bytes(const llmhip_scck_info& c) {
  const u128 t = c.context_len, h = c.hidden_dim, f = ffn_dim(c.hidden_dim);
  const u128 band = c.local_window < c.context_len ? c.local_window : c.context_len;
  const u128 kv = (u128)c.num_kv_heads * (c.hidden_dim / c.num_heads);
  const u128 per_layer = 6 * t * h + 2 * t * kv + 2 * t * f + (u128)c.num_heads * t * band + 2 * t;
  const u128 shared = 3 * t * h + 2 * t * c.vocab_size + 6 * t * h + 3 * t * f;
  return ((u128)c.num_layers * per_layer + shared) * 4;
}

// config.rs:169-217 (ModelConfig::validate), as the message from_bytes
// wraps it in (checkpoint.rs:209).
bool validate(const llmhip_scck_info& c, std::string& err) {
  char buf[200];
  auto small = [&](const char* field, uint64_t min) {
    snprintf(buf, sizeof buf, "checkpoint config is invalid: %s must be at least %llu", field,
             (unsigned long long)min);
    err = buf;
    return false;
  };
  if (c.num_layers == 0) return small("num_layers", 1);
  if (c.hidden_dim < 8) return small("hidden_dim", 8);
  if (c.num_heads == 0) return small("num_heads", 1);
  if (c.context_len < 2) return small("context_len", 2);
  if (c.local_window == 0) return small("local_window", 1);
  if (c.vocab_size < kFirstMergeId) return small("vocab_size", kFirstMergeId);
  if (c.hidden_dim % c.num_heads != 0) {
    snprintf(buf, sizeof buf, "checkpoint config is invalid: num_heads %u must divide hidden_dim %u", c.num_heads,
             c.hidden_dim);
    err = buf;
    return false;
  }
  const uint32_t head_dim = c.hidden_dim / c.num_heads;
  if (head_dim % 2 != 0) {
    snprintf(buf, sizeof buf, "checkpoint config is invalid: head_dim %u must be even", head_dim);
    err = buf;
    return false;
  }
  if (c.num_kv_heads == 0) return small("num_kv_heads", 1);
  if (c.num_heads % c.num_kv_heads != 0) {
    snprintf(buf, sizeof buf, "checkpoint config is invalid: num_kv_heads %u must divide num_heads %u",
             c.num_kv_heads, c.num_heads);
    err = buf;
    return false;
  }
  // config.rs:209 tests `rope_theta <= 1.0`, which a NaN passes: such a
  // file is accepted, as Checkpoint::from_bytes accepts it.
  if (c.rope_theta <= 1.0f) return small("rope_theta", 2);
  const u128 training = param_count(c) * 4 * 4 + activation_bytes(c);  // config.rs:346-355
  if (training > kMaxTrainingBytes) {
    snprintf(buf, sizeof buf, "checkpoint config is invalid: needs more than %llu bytes to train",
             (unsigned long long)kMaxTrainingBytes);
    err = buf;
    return false;
  }
  return true;
}

bool parse(const uint8_t* bytes, size_t len, llmhip_scck_info* o, std::string& err) {
  memset(o, 0, sizeof *o);
  Reader r{bytes, len, 0};
  const uint8_t* p;
  if (!r.take(4, &p, err) || memcmp(p, "SCCK", 4) != 0) {
    err = "not a scriptonait checkpoint";
    return false;
  }
  if (!r.u32(&o->version, err)) return false;
  if (o->version < kMinVersion || o->version > kVersion) {
    char buf[120];
    snprintf(buf, sizeof buf, "checkpoint format version %u, expected %u to %u", o->version, kMinVersion, kVersion);
    err = buf;
    return false;
  }
  uint32_t* shape[7] = {&o->num_layers, &o->hidden_dim, &o->num_heads, &o->num_kv_heads,
                        &o->context_len, &o->local_window, &o->vocab_size};
  for (uint32_t* f : shape)
    if (!r.u32(f, err)) return false;
  if (!r.f32(&o->rope_theta, err)) return false;
  if (!r.u32(&o->use_ple, err)) return false;
  o->use_ple = o->use_ple != 0;
  if (!validate(*o, err)) return false;
  if (!r.u64(&o->step, err)) return false;
  o->tokens_seen = 0;  // absent before v3 (checkpoint.rs:213-215)
  if (o->version >= 3 && !r.u64(&o->tokens_seen, err)) return false;
  o->planned_steps = 0;  // absent before v4 (checkpoint.rs:216-220)
  o->plateau_scale = 1.0f;
  if (o->version >= 4 && (!r.u32(&o->planned_steps, err) || !r.f32(&o->plateau_scale, err))) return false;
  if (!r.u32(&o->weight_dtype, err)) return false;
  if (o->weight_dtype > 1) {
    err = "unknown weight dtype " + std::to_string(o->weight_dtype);
    return false;
  }
  // The tokenizer (tokenizer.rs:360-390).
  uint32_t tlen;
  if (!r.u32(&tlen, err)) return false;
  o->tokenizer_offset = r.at;
  o->tokenizer_bytes = tlen;
  const uint8_t* t;
  if (!r.take(tlen, &t, err)) return false;
  if (tlen < 12 || memcmp(t, "SCTK", 4) != 0) {
    err = "not a scriptonait tokenizer file";
    return false;
  }
  uint32_t tver, nmerge;
  memcpy(&tver, t + 4, 4);
  memcpy(&nmerge, t + 8, 4);
  if (tver != 1) {
    err = "tokenizer format version " + std::to_string(tver) + ", expected 1";
    return false;
  }
  if ((uint64_t)tlen != 12 + (uint64_t)nmerge * 8) {
    err = "expected " + std::to_string(12 + (uint64_t)nmerge * 8) + " bytes for " + std::to_string(nmerge) +
          " merges, got " + std::to_string(tlen);
    return false;
  }
  for (uint32_t i = 0; i < nmerge; ++i) {
    uint32_t a, b;
    memcpy(&a, t + 12 + (size_t)i * 8, 4);
    memcpy(&b, t + 16 + (size_t)i * 8, 4);
    const uint32_t limit = kFirstMergeId + i;
    if (a >= limit || b >= limit) {
      err = "merge " + std::to_string(i) + " refers to token id >= " + std::to_string(limit);
      return false;
    }
  }
  o->num_merges = nmerge;
  const uint64_t tok_vocab = (uint64_t)kFirstMergeId + nmerge;
  if (tok_vocab != o->vocab_size) {
    err = "checkpoint is inconsistent: config says vocab_size " + std::to_string(o->vocab_size) +
          ", its tokenizer has " + std::to_string(tok_vocab);
    return false;
  }
  // The weights.
  uint32_t wlen;
  if (!r.u32(&wlen, err)) return false;
  o->weights_offset = r.at;
  o->weights_bytes = wlen;
  const uint8_t* w;
  if (!r.take(wlen, &w, err)) return false;
  o->param_count = (uint64_t)param_count(*o);  // below 2^27 once validate passed
  if (o->weight_dtype == 1 && wlen % 2 != 0) {
    err = "bf16 weights have an odd byte count";
    return false;
  }
  const uint64_t widened = o->weight_dtype == 1 ? (uint64_t)wlen * 2 : wlen;
  if (widened != o->param_count * 4) {
    err = "expected " + std::to_string(o->param_count * 4) + " bytes for this config, got " + std::to_string(widened);
    return false;
  }
  return true;
}

}  // namespace

extern "C" {

int llmhip_scck_parse(const uint8_t* bytes, size_t len, llmhip_scck_info* out) {
  if (!out || (!bytes && len)) {
    llmhip::set_last_error("bytes and out are required");
    return LLMHIP_ERR_INVALID_ARGUMENT;
  }
  std::string err;
  if (!parse(bytes, len, out, err)) {
    llmhip::set_last_error(err);
    return LLMHIP_ERR_INVALID_ARGUMENT;
  }
  return LLMHIP_OK;
}

int llmhip_scck_read_params(const uint8_t* bytes, size_t len, const llmhip_scck_info* info, uint64_t first,
                            uint64_t count, float* out) {
  if (!bytes || !info || (count && !out)) {
    llmhip::set_last_error("bytes, info and out are required");
    return LLMHIP_ERR_INVALID_ARGUMENT;
  }
  if (first > info->param_count || count > info->param_count - first) {
    llmhip::set_last_error("parameter range past the checkpoint's parameters");
    return LLMHIP_ERR_INVALID_ARGUMENT;
  }
  const uint64_t width = info->weight_dtype == 1 ? 2 : 4;
  if (info->weights_offset > len || info->param_count * width > len - info->weights_offset) {
    llmhip::set_last_error("info does not describe these bytes");
    return LLMHIP_ERR_INVALID_ARGUMENT;
  }
  const uint8_t* w = bytes + info->weights_offset + first * width;
  if (width == 4) {
    memcpy(out, w, count * 4);
  } else {
    for (uint64_t i = 0; i < count; ++i) {  // bf16.rs:22-25: the bits are an f32 prefix
      uint16_t b;
      memcpy(&b, w + i * 2, 2);
      const uint32_t bits = (uint32_t)b << 16;
      memcpy(out + i, &bits, 4);
    }
  }
  return LLMHIP_OK;
}

}  // extern "C"
