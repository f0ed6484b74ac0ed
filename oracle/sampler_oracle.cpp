// CPU ORACLE — test infrastructure only, never the product path.
//
// A line-by-line C++17 restatement of scriptonait's decode-time sampler,
// used (1) by tests/ as the parity checker for the HIP library and (2) by
// bench.py's cpu_baseline leg as the timed CPU baseline. Nothing in the
// shipped library (scriptonait_amd/) links, loads or calls this file.
//
// Reference (all paths relative to the scriptonait repository):
//   crates/llm-core/src/ops/linear.rs:19-32, 110-125  `dot`, `linear_fwd`
//                                            (the tied output head's logits)
//   crates/llm-core/src/rng.rs:11-34        SplitMix64 `Rng`
//   crates/llm-core/src/ops/loss.rs:5-16     `argmax` (greedy tie-break)
//   crates/llm-core/src/generate.rs:325-420  `sample_with`
//   crates/llm-core/src/tokenizer.rs:38      EOS = 258 (passed in as eos_id)
//
// Arithmetic rules that make this a faithful restatement:
//   * binary32 everywhere the reference uses f32, built with -O2, no
//     fast-math and -ffp-contract=off (no fused multiply-adds);
//   * `f32::exp` is glibc `expf` (what Rust links on x86_64-linux-gnu);
//   * every f32 sum is a sequential left fold in sorted order, as
//     `Iterator::sum` and the explicit loops in the reference are;
//   * the sort is the reference's total order: value descending, ties by
//     ascending id. `partial_cmp` makes -0.0 == +0.0. NaN is the one input
//     where the reference's comparator is not a total order (pdqsort's
//     output then depends on its internals); here NaN sorts last. Rows
//     holding NaN after masking are "parity unpinned".
//
// Parity pinning of this file (see tests/test_oracle.py):
//   * SplitMix64 against Vigna's published output for seed 0 and the closed
//     form state_n = seed + n * 0x9E3779B97F4A7C15;
//   * the seven sampler property tests of generate.rs:550-692 and the PRNG
//     tests of rng.rs:48-91;
//   * closed forms (top_k = 1 and greedy give argmax; flat logits make the
//     draw index floor(u * n)); brute force over all 2^24 draws for tiny
//     rows (each id's share of draws equals its f32 probability mass);
//   * an independent pure-Python restatement on small random rows;
//   * linear_fwd: one-hot rows give the weight column exactly, small
//     integers give the exact integer dot product, and rows built so that
//     the four-accumulator order, a sequential fold and a pairwise sum give
//     three different binary32 results pin the order.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

extern "C" {

typedef struct llmhip_params {
  float temperature;
  uint32_t top_k;
  float top_p;
  float min_p;
  float repetition_penalty;
} llmhip_params;

// crates/llm-core/src/ops/linear.rs:19-32 (`dot`), as linear_fwd
// (linear.rs:110-125, through dot_block :83-91) calls it for every (row,
// output): four accumulators over the chunks of 4 (acc[k] += a[4j+k] *
// b[4j+k], a separate binary32 multiply and add, in increasing j), then the
// remainder's products as a left fold, then ((acc0 + acc1) + (acc2 + acc3))
// + tail. Rust's f32 `Sum` starts its fold from a zero whose sign some
// toolchains take as -0.0; the two starts differ only in the sign of an
// all-zero tail, which leaves every nonzero result and every zero's value
// unchanged. y is [rows][out_dim]; w is [out_dim][in_dim] (the tied head's
// `embed`, model.rs:396-397).
static float dot4(const float* a, const float* b, size_t n) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const size_t n4 = n / 4 * 4;
  for (size_t j = 0; j < n4; j += 4) {
    for (int k = 0; k < 4; ++k) {
      const float prod = a[j + k] * b[j + k];
      acc[k] = acc[k] + prod;
    }
  }
  float tail = 0.0f;
  for (size_t j = n4; j < n; ++j) {
    const float prod = a[j] * b[j];
    tail = tail + prod;
  }
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + tail;
}

void oracle_linear_fwd(const float* x, const float* w, size_t rows, size_t in_dim, size_t out_dim, float* y,
                       int threads) {
  auto work = [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r)
      for (size_t o = 0; o < out_dim; ++o) y[r * out_dim + o] = dot4(x + r * in_dim, w + o * in_dim, in_dim);
  };
  if (threads <= 1 || rows < 2) {
    work(0, rows);
    return;
  }
  std::vector<std::thread> pool;
  const size_t per = (rows + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const size_t r0 = std::min(rows, t * per), r1 = std::min(rows, r0 + per);
    if (r0 < r1) pool.emplace_back(work, r0, r1);
  }
  for (auto& th : pool) th.join();
}

// rng.rs:16-22
uint64_t oracle_splitmix64_next(uint64_t* state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// rng.rs:31-34
float oracle_next_f32(uint64_t* state) {
  return (float)(oracle_splitmix64_next(state) >> 40) / (float)(1u << 24);
}

// ops/loss.rs:6-16
uint32_t oracle_argmax(const float* row, size_t n) {
  size_t best = 0;
  float best_val = -INFINITY;
  for (size_t i = 0; i < n; ++i) {
    if (row[i] > best_val) {
      best_val = row[i];
      best = i;
    }
  }
  return (uint32_t)best;
}

// generate.rs:325-420. `out_probs` (nullable) receives the post-truncation
// probabilities scattered by id (zeros elsewhere), `out_kept` the number of
// candidates the draw walked over (0 on the greedy and degenerate exits), and
// `out_margin` the smallest gap between the two operands of any comparison
// that decided min-p, top-p or the draw (+inf when nothing was decided).
uint32_t oracle_sample_with(const float* logits, size_t V, const llmhip_params* prm,
                            const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                            const uint32_t* recent, size_t H, uint64_t* rng_state,
                            float* out_probs, uint32_t* out_kept, float* out_margin) {
  if (out_probs) memset(out_probs, 0, V * sizeof(float));
  if (out_kept) *out_kept = 0;
  if (out_margin) *out_margin = INFINITY;

  // generate.rs:331
  std::vector<float> work(logits, logits + V);

  // generate.rs:333-341: masked ids become -inf; EOS and ids past the end of
  // the mask stay allowed.
  if (allowed) {
    for (size_t id = 0; id < V; ++id) {
      if ((uint32_t)id != eos_id && id < allowed_len && !allowed[id]) work[id] = -INFINITY;
    }
  }

  // generate.rs:343-352: once per occurrence, in history order.
  const float rp = prm->repetition_penalty;
  if (rp != 1.0f) {
    for (size_t j = 0; j < H; ++j) {
      const size_t id = recent[j];
      if (id < V) {
        const float l = work[id];
        work[id] = l > 0.0f ? l / rp : l * rp;
      }
    }
  }

  // generate.rs:354-356
  if (prm->temperature <= 0.0f) return oracle_argmax(work.data(), V);
  // generate.rs:357-359
  for (size_t i = 0; i < V; ++i) work[i] /= prm->temperature;

  // generate.rs:364-367: value descending, ties by ascending id.
  std::vector<uint32_t> order(V);
  for (size_t i = 0; i < V; ++i) order[i] = (uint32_t)i;
  std::sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
    const float wa = work[a], wb = work[b];
    const bool na = wa != wa, nb = wb != wb;
    if (na || nb) {
      if (na && nb) return a < b;
      return nb;  // NaN last
    }
    if (wa > wb) return true;
    if (wa < wb) return false;
    return a < b;
  });
  // generate.rs:368-370
  size_t n = V;
  if (prm->top_k > 0 && prm->top_k < n) n = prm->top_k;

  // generate.rs:372-377
  float mx = -INFINITY;
  for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, work[order[i]]);
  std::vector<float> probs(n);
  for (size_t i = 0; i < n; ++i) probs[i] = expf(work[order[i]] - mx);
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += probs[i];
  if (sum <= 0.0f || !isfinite(sum)) return n > 0 ? order[0] : 0u;
  // generate.rs:378-380
  for (size_t i = 0; i < n; ++i) probs[i] /= sum;

  float margin = INFINITY;
  // generate.rs:384-395
  if (prm->min_p > 0.0f) {
    const float threshold = prm->min_p * (n > 0 ? probs[0] : 0.0f);
    size_t keep = 0;
    while (keep < n) {
      margin = fminf(margin, fabsf(probs[keep] - threshold));
      if (!(probs[keep] >= threshold)) break;
      ++keep;
    }
    if (keep < 1) keep = 1;
    n = std::min(n, keep);
  }
  // generate.rs:397-409
  if (prm->top_p < 1.0f) {
    float cumulative = 0.0f;
    size_t keep = n;
    for (size_t i = 0; i < n; ++i) {
      cumulative += probs[i];
      margin = fminf(margin, fabsf(cumulative - prm->top_p));
      if (cumulative >= prm->top_p) {
        keep = i + 1;
        break;
      }
    }
    n = keep;
  }
  // generate.rs:411-419
  float total = 0.0f;
  for (size_t i = 0; i < n; ++i) total += probs[i];
  if (out_kept) *out_kept = (uint32_t)n;
  if (out_probs) {
    for (size_t i = 0; i < n; ++i) out_probs[order[i]] = probs[i];
  }
  float r = oracle_next_f32(rng_state) * total;
  for (size_t i = 0; i < n; ++i) {
    margin = fminf(margin, fabsf(r - probs[i]));
    if (r < probs[i]) {
      if (out_margin) *out_margin = margin;
      return order[i];
    }
    r -= probs[i];
  }
  if (out_margin) *out_margin = margin;
  return n > 0 ? order[n - 1] : 0u;
}

// Batched form with the same argument meaning as llmhip_sample_host: rows
// are `ld` floats apart, `params` is shared when params_stride == 0, the
// history of row b is hist[hist_offsets[b] .. hist_offsets[b+1]), and
// rng_state[b] is read and advanced in place. Rows are split statically
// over `threads` std::threads (1 = the reference's sequential use).
int oracle_sample_batch(const float* logits, size_t B, size_t V, size_t ld,
                        const llmhip_params* params, size_t params_stride,
                        const uint32_t* hist, const uint32_t* hist_offsets,
                        const uint8_t* allowed, size_t allowed_len, uint32_t eos_id,
                        uint64_t* rng_state, uint32_t* out_ids, float* out_probs,
                        uint32_t* out_kept, float* out_margin, int threads) {
  if (ld < V) return -1;
  auto run = [&](size_t lo, size_t hi) {
    for (size_t b = lo; b < hi; ++b) {
      const llmhip_params* p = params + b * params_stride;
      const uint32_t* h = hist ? hist + hist_offsets[b] : nullptr;
      const size_t H = hist ? (size_t)(hist_offsets[b + 1] - hist_offsets[b]) : 0;
      out_ids[b] = oracle_sample_with(logits + b * ld, V, p, allowed, allowed_len, eos_id, h, H,
                                      &rng_state[b], out_probs ? out_probs + b * V : nullptr,
                                      out_kept ? out_kept + b : nullptr,
                                      out_margin ? out_margin + b : nullptr);
    }
  };
  if (threads <= 1 || B <= 1) {
    run(0, B);
    return 0;
  }
  std::vector<std::thread> pool;
  const size_t T = std::min<size_t>((size_t)threads, B);
  for (size_t t = 0; t < T; ++t) {
    const size_t lo = B * t / T, hi = B * (t + 1) / T;
    pool.emplace_back(run, lo, hi);
  }
  for (auto& th : pool) th.join();
  return 0;
}

}  // extern "C"
