// ref_driver.cpp -- C entry points around the reference's own
// cudaforge::scheduler::SpeculativeEngine (csrc/src/scheduler/speculative.cpp,
// csrc/include/cudaforge/scheduler/speculative.h), compiled from the sources
// where they lie under /root/reference into oracle/_ref/libref_spec.so.
//
// TEST INFRASTRUCTURE ONLY: used to pin the C oracle (spec_oracle.c) and to
// write golden fixtures; never linked into the product library.
#include <cstdint>
#include <random>
#include <stdexcept>
#include <vector>

#include "cudaforge/scheduler/speculative.h"

using cudaforge::scheduler::SpeculativeConfig;
using cudaforge::scheduler::SpeculativeEngine;
using cudaforge::scheduler::SpeculativeVerificationResult;

extern "C" {

// The uniform stream the reference engine draws from: rng_(rng_seed)
// (speculative.cpp:8-9) and uniform_real_distribution<float>(0, 1)
// (speculative.cpp:13-14, 64, 72).
int ref_uniforms(uint64_t seed, int n, float *out) {
  std::mt19937 rng(seed);
  std::uniform_real_distribution<float> dist(0.0f, 1.0f);
  for (int i = 0; i < n; ++i) out[i] = dist(rng);
  return 0;
}

// `ncalls` successive calls on ONE engine seeded with `seed` (so the RNG
// stream carries over between calls, as it does for a long-lived engine).
// tokens [ncalls, K]; dprobs [ncalls, K, V]; tprobs [ncalls, K+1, V].
// out_tokens [ncalls, K] (accepted tokens, -1 padded).
// Returns 0, or -1 when the reference threw std::invalid_argument.
int ref_verify(uint64_t seed, int greedy, int ncalls, int K, int64_t V,
               const int32_t *tokens, const float *dprobs, const float *tprobs,
               int32_t eos, int32_t *out_tokens, int32_t *out_num_acc,
               int32_t *out_final, int32_t *out_eos) {
  SpeculativeConfig cfg;
  cfg.rng_seed = seed;
  SpeculativeEngine eng(cfg);
  for (int c = 0; c < ncalls; ++c) {
    std::vector<int32_t> toks(tokens + (int64_t)c * K, tokens + (int64_t)(c + 1) * K);
    std::vector<std::vector<float>> d(K), t(K + 1);
    for (int i = 0; i < K; ++i)
      d[i].assign(dprobs + ((int64_t)c * K + i) * V, dprobs + ((int64_t)c * K + i + 1) * V);
    for (int i = 0; i <= K; ++i)
      t[i].assign(tprobs + ((int64_t)c * (K + 1) + i) * V,
                  tprobs + ((int64_t)c * (K + 1) + i + 1) * V);
    SpeculativeVerificationResult r;
    try {
      r = greedy ? eng.verify_candidates_greedy(toks, t, eos)
                 : eng.verify_candidates(toks, d, t, eos);
    } catch (const std::invalid_argument &) {
      return -1;
    }
    for (int i = 0; i < K; ++i)
      out_tokens[(int64_t)c * K + i] = i < (int)r.accepted_tokens.size() ? r.accepted_tokens[i] : -1;
    out_num_acc[c] = (int32_t)r.num_accepted;
    out_final[c] = r.final_token;
    out_eos[c] = r.end_of_sequence ? 1 : 0;
  }
  return 0;
}

}  // extern "C"
