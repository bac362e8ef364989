/*
 * spec_oracle.h -- CPU oracle for the speculative-decoding verification path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links or calls
 * this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg use it, and only as the checker / CPU baseline.
 *
 * Plain C99 restatement of the reference algorithms (citations are
 * path:line inside Bahaa-Labs/CUDAForge):
 *   - cpp semantics  : csrc/src/scheduler/speculative.cpp:11-150
 *   - python semantics: cudaforge/speculative.py:57-211 with caller-supplied
 *     uniforms in place of torch.rand_like / torch.multinomial
 *   - tree semantics : multi-candidate rejection sampling (SpecInfer) that
 *     reduces to the cpp semantics on a one-child chain.
 *
 * All arithmetic that the reference performs in fp32 is performed here in
 * fp32, in the same order, with no contraction (built with -ffp-contract=off).
 */
#ifndef SPEC_ORACLE_H
#define SPEC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads used by the OpenMP loops of the batched functions. */
void orc_set_threads(int n);

/* speculative.cpp:11-24 -- sequential fp32 inverse CDF. */
int32_t orc_sample_from_distribution(const float *probs, int64_t V, float r);

/* speculative.cpp:26-48 -- residual max(0, t - d), sequential fp32 sum,
 * fallback to t when sum <= 1e-6f, per-element division, inverse CDF.
 * *fallback (optional) receives 1 when the fallback branch was taken. */
int32_t orc_sample_adjusted(const float *target_p, const float *draft_q,
                            int64_t V, float r, int *fallback);

/* Sequential fp32 sum of a row, exactly as speculative.cpp:30-35 forms it. */
float orc_seq_sum(const float *x, int64_t V);

/* speculative.cpp:50-103 for one sequence, uniforms supplied in the order the
 * reference draws them from its mt19937 (one per acceptance test, then one
 * for the final sample).  Row i of dprobs/tprobs starts at i*ld.
 * Returns 0, or -1 on the size errors the reference throws on, or -2 on an
 * out-of-range token.  out_tokens receives the accepted draft tokens. */
int orc_verify_cpp(int K, int64_t V, int64_t ld, const int32_t *tokens,
                   const float *dprobs, const float *tprobs, int32_t eos,
                   const float *U, int32_t *out_tokens, int32_t *out_num_acc,
                   int32_t *out_final, int32_t *out_eos, int32_t *out_draws);

/* speculative.cpp:105-150 (greedy; first maximum as std::max_element). */
int orc_verify_greedy(int K, int64_t V, int64_t ld, const int32_t *tokens,
                      const float *tprobs, int32_t eos, int32_t *out_tokens,
                      int32_t *out_num_acc, int32_t *out_final,
                      int32_t *out_eos);

/* First index of the maximum, as std::max_element + std::distance. */
int32_t orc_argmax_first(const float *x, int64_t V);

/* Batched cpp-mode verification over B rows (OpenMP over rows).
 * tprobs row (b,i) at b*tsb + i*ld, dprobs row (b,i) at b*dsb + i*ld,
 * tokens (b,i) at b*K+i, uniforms (b,j) at b*(K+1)+j.
 * greedy != 0 selects verify_candidates_greedy.
 * out_tokens is [B, K+1]: accepted drafts followed by the final token (the
 * final token is not repeated after an accepted EOS). */
int orc_chain_verify_batch(int B, int K, int64_t V, int64_t ld, int64_t tsb,
                           int64_t dsb, const float *tprobs,
                           const float *dprobs, const int32_t *tokens,
                           const float *U, int32_t eos, int greedy,
                           int32_t *out_accept_len, int32_t *out_tokens,
                           int32_t *out_num_emitted, int32_t *out_final,
                           int32_t *out_eos);

/* Row softmax of logits / T in fp32 (max, exp, fp64 sum, divide); used by
 * the CPU baseline only.  x and p may alias. */
void orc_softmax_rows(const float *x, float *p, int64_t rows, int64_t V,
                      int64_t ld, float temperature);

/* python-mode semantics of speculative.py:152-195 over a batch with fed
 * uniforms U [B, K+2]: columns 0..K-1 replace rand_like at :161, column K
 * drives the resample (:182) or the bonus draw (:189), column K+1 the bonus
 * that follows a rejection at the last position (n = K - 1 makes the
 * reference's num_accepted equal K, so :188 appends a bonus too).  The bonus
 * is drawn from row K after the top-p filter of :67-81.  out_tokens is
 * [B, K+1], -1 padded; *out_n receives the batch accept count n (accepted
 * drafts) and *out_num_emitted the tokens per row (the reference's
 * num_accepted: n + 1, or K + 1 after a rejection at K - 1). */
int orc_verify_python(int B, int K, int64_t V, int64_t ld, int64_t tsb,
                      int64_t dsb, const float *tprobs, const float *dprobs,
                      const int32_t *tokens, const float *U, float top_p,
                      int32_t *out_n, int32_t *out_num_emitted,
                      int32_t *out_tokens);

/* The normalised weights the python-mode resample draws from (the residual,
 * or the target row on the sum <= 1e-6 fallback; returns 1 on fallback). */
int orc_py_residual_weights(const float *target_p, const float *draft_q,
                            int64_t V, float *out);
/* The normalised weights the python-mode bonus draws from (top-p kept
 * target probabilities over their sequential fp32 sum). */
void orc_py_bonus_weights(const float *pk, int64_t V, float top_p, float *out);
/* The python-mode residual draw (speculative.py:171-182): the weights of
 * orc_py_residual_weights drawn with the python-mode inverse CDF. */
int32_t orc_py_sample_adjusted(const float *target_p, const float *draft_q,
                               int64_t V, float u, int *fallback);

/* Top-p keep set (speculative.py:67-81) restated without a sort: token j is
 * kept iff the probability mass strictly above p_j is <= top_p (fp64 sums).
 * For distinct probabilities this equals the reference's shifted-cumsum rule;
 * tied probabilities are kept or dropped together. */
void orc_topp_keep(const float *p, int64_t V, float top_p, uint8_t *keep);

/* Python-mode draw from unnormalised non-negative weights (the bonus and the
 * filtered sampler): sequential fp32 sum, per-element division, then the
 * first i whose sequential fp32 prefix sum exceeds u (and is >= FLT_MIN);
 * past the end of the sums, the last index of positive weight.  A
 * zero-weight index is never returned (as torch.multinomial). */
int32_t orc_sample_weights(const float *w, int64_t V, float u);

/* Tree verification (multi-candidate rejection sampling), cpp semantics.
 * parent[0] = -1, parent[i] < i.  Row n of tprobs/dprobs is node n's target
 * and draft distribution over the next token.  Children of a node are tested
 * in increasing index order; every test and the final draw consume the next
 * uniform of U (length n_u).  Greedy: a child is accepted iff its token is the
 * first argmax of the parent's target row.
 * out_path receives the accepted node ids starting with the root (0);
 * *out_path_len = 1 + accepted drafts. Returns 0, -1 if uniforms ran out. */
int orc_tree_verify(int N, int64_t V, int64_t ld, const int32_t *parent,
                    const int32_t *tok, const float *tprobs,
                    const float *dprobs, int32_t eos, const float *U, int n_u,
                    int greedy, int32_t *out_path, int32_t *out_path_len,
                    int32_t *out_final, int32_t *out_eos, int32_t *out_draws);

#ifdef __cplusplus
}
#endif

#endif /* SPEC_ORACLE_H */
