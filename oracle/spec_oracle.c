/*
 * spec_oracle.c -- CPU oracle for the speculative-decoding verification path.
 *
 * TEST INFRASTRUCTURE ONLY (see spec_oracle.h).  Build with
 * -ffp-contract=off so that every fp32 operation rounds exactly where the
 * reference's does.
 */
#include "spec_oracle.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* Threads of the OpenMP loops below (the CPU baseline times 1 and all). */
void orc_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}

/* speculative.cpp:11-24: cumulative += probs[i]; if (r <= cumulative) return i;
 * falls through to the last index. */
int32_t orc_sample_from_distribution(const float *probs, int64_t V, float r) {
  float cumulative = 0.0f;
  for (int64_t i = 0; i < V; ++i) {
    cumulative += probs[i];
    if (r <= cumulative) return (int32_t)i;
  }
  return (int32_t)(V - 1);
}

float orc_seq_sum(const float *x, int64_t V) {
  float s = 0.0f;
  for (int64_t i = 0; i < V; ++i) s += x[i];
  return s;
}

/* std::max(0.0f, v) is (0.0f < v) ? v : 0.0f. */
static inline float relu_std_max(float v) { return (0.0f < v) ? v : 0.0f; }

/* speculative.cpp:26-48 */
int32_t orc_sample_adjusted(const float *target_p, const float *draft_q,
                            int64_t V, float r, int *fallback) {
  float *adjusted = (float *)malloc((size_t)V * sizeof(float));
  float sum = 0.0f;
  for (int64_t i = 0; i < V; ++i) {
    adjusted[i] = relu_std_max(target_p[i] - draft_q[i]);
    sum += adjusted[i];
  }
  if (sum <= 1e-6f) {
    free(adjusted);
    if (fallback) *fallback = 1;
    return orc_sample_from_distribution(target_p, V, r);
  }
  if (fallback) *fallback = 0;
  for (int64_t i = 0; i < V; ++i) adjusted[i] /= sum;
  int32_t tok = orc_sample_from_distribution(adjusted, V, r);
  free(adjusted);
  return tok;
}

/* std::max_element returns the first largest element (operator<). */
int32_t orc_argmax_first(const float *x, int64_t V) {
  int64_t best = 0;
  for (int64_t i = 1; i < V; ++i)
    if (x[best] < x[i]) best = i;
  return (int32_t)best;
}

/* speculative.cpp:50-103 with the mt19937 draws replaced by U[0..]. */
int orc_verify_cpp(int K, int64_t V, int64_t ld, const int32_t *tokens,
                   const float *dprobs, const float *tprobs, int32_t eos,
                   const float *U, int32_t *out_tokens, int32_t *out_num_acc,
                   int32_t *out_final, int32_t *out_eos, int32_t *out_draws) {
  int draws = 0, n = 0;
  *out_eos = 0;
  *out_final = -1;
  for (int i = 0; i < K; ++i) {
    int32_t tok = tokens[i];
    if (tok < 0 || tok >= V) return -2;
    float q = dprobs[i * ld + tok]; /* draft prob, :68 */
    float p = tprobs[i * ld + tok]; /* target prob, :69 */
    float ratio = (q > 0.0f) ? ((1.0f < p / q) ? 1.0f : p / q) : 0.0f; /* :71 */
    float r = U[draws++];                                               /* :72 */
    if (r <= ratio) {                                                   /* :74 */
      out_tokens[n++] = tok;
      if (tok == eos) {
        *out_eos = 1;
        *out_final = eos;
        *out_num_acc = n;
        *out_draws = draws;
        return 0;
      }
    } else {
      *out_final = orc_sample_adjusted(tprobs + i * ld, dprobs + i * ld, V,
                                       U[draws++], NULL);
      *out_eos = (*out_final == eos);
      *out_num_acc = n;
      *out_draws = draws;
      return 0;
    }
  }
  *out_final = orc_sample_from_distribution(tprobs + (int64_t)K * ld, V,
                                            U[draws++]); /* :97 */
  *out_eos = (*out_final == eos);
  *out_num_acc = n;
  *out_draws = draws;
  return 0;
}

/* speculative.cpp:105-150 */
int orc_verify_greedy(int K, int64_t V, int64_t ld, const int32_t *tokens,
                      const float *tprobs, int32_t eos, int32_t *out_tokens,
                      int32_t *out_num_acc, int32_t *out_final,
                      int32_t *out_eos) {
  int n = 0;
  *out_eos = 0;
  for (int i = 0; i < K; ++i) {
    int32_t tok = tokens[i];
    int32_t am = orc_argmax_first(tprobs + i * ld, V);
    if (tok == am) {
      out_tokens[n++] = tok;
      if (tok == eos) {
        *out_eos = 1;
        *out_final = eos;
        *out_num_acc = n;
        return 0;
      }
    } else {
      *out_final = am;
      *out_eos = (am == eos);
      *out_num_acc = n;
      return 0;
    }
  }
  *out_final = orc_argmax_first(tprobs + (int64_t)K * ld, V);
  *out_eos = (*out_final == eos);
  *out_num_acc = n;
  return 0;
}

int orc_chain_verify_batch(int B, int K, int64_t V, int64_t ld, int64_t tsb,
                           int64_t dsb, const float *tprobs,
                           const float *dprobs, const int32_t *tokens,
                           const float *U, int32_t eos, int greedy,
                           int32_t *out_accept_len, int32_t *out_tokens,
                           int32_t *out_num_emitted, int32_t *out_final,
                           int32_t *out_eos) {
  int err = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : err)
  for (int b = 0; b < B; ++b) {
    int32_t n = 0, fin = -1, eflag = 0, draws = 0;
    int32_t *row_out = out_tokens + (int64_t)b * (K + 1);
    for (int j = 0; j <= K; ++j) row_out[j] = -1;
    int rc;
    if (greedy)
      rc = orc_verify_greedy(K, V, ld, tokens + (int64_t)b * K,
                             tprobs + b * tsb, eos, row_out, &n, &fin, &eflag);
    else
      rc = orc_verify_cpp(K, V, ld, tokens + (int64_t)b * K, dprobs + b * dsb,
                          tprobs + b * tsb, eos, U + (int64_t)b * (K + 1),
                          row_out, &n, &fin, &eflag, &draws);
    if (rc) err |= 1;
    /* An accepted EOS ends the step with final_token == eos already present
     * as the last accepted token (speculative.cpp:79-83); it is emitted once. */
    int eos_accepted = (n > 0 && row_out[n - 1] == eos);
    out_accept_len[b] = n;
    out_final[b] = fin;
    out_eos[b] = eflag;
    out_num_emitted[b] = eos_accepted ? n : n + 1;
    if (!eos_accepted) row_out[n] = fin;
  }
  return err ? -2 : 0;
}

void orc_softmax_rows(const float *x, float *p, int64_t rows, int64_t V,
                      int64_t ld, float temperature) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * ld;
    float *pr = p + r * ld;
    float m = -INFINITY;
    for (int64_t i = 0; i < V; ++i) {
      float a = xr[i] / temperature;
      if (a > m) m = a;
    }
    double s = 0.0;
    for (int64_t i = 0; i < V; ++i) {
      float e = expf(xr[i] / temperature - m);
      pr[i] = e;
      s += e;
    }
    float inv = (float)(1.0 / s);
    for (int64_t i = 0; i < V; ++i) pr[i] = pr[i] * inv;
  }
}

/* ---- python semantics (speculative.py) ---------------------------------- */

typedef struct {
  float p;
  int64_t i;
} pidx_t;

static int cmp_desc(const void *a, const void *b) {
  float x = ((const pidx_t *)a)->p, y = ((const pidx_t *)b)->p;
  if (x > y) return -1;
  if (x < y) return 1;
  int64_t i = ((const pidx_t *)a)->i, j = ((const pidx_t *)b)->i;
  return (i < j) ? -1 : (i > j);
}

void orc_topp_keep(const float *p, int64_t V, float top_p, uint8_t *keep) {
  if (!(top_p < 1.0f)) { /* speculative.py:67: no filtering at top_p >= 1 */
    for (int64_t i = 0; i < V; ++i) keep[i] = 1;
    return;
  }
  pidx_t *s = (pidx_t *)malloc((size_t)V * sizeof(pidx_t));
  for (int64_t i = 0; i < V; ++i) {
    s[i].p = p[i];
    s[i].i = i;
  }
  qsort(s, (size_t)V, sizeof(pidx_t), cmp_desc);
  double above = 0.0; /* mass strictly above the current value group */
  int64_t g = 0;
  while (g < V) {
    int64_t h = g;
    double grp = 0.0;
    while (h < V && s[h].p == s[g].p) grp += s[h++].p;
    uint8_t k = (above <= (double)top_p) ? 1 : 0;
    if (g == 0) k = 1; /* :76 the top token is always kept */
    for (int64_t j = g; j < h; ++j) keep[s[j].i] = k;
    above += grp;
    g = h;
  }
  free(s);
}

/* Python-mode inverse CDF: the first i whose sequential fp32 prefix sum
 * exceeds u (and is at least FLT_MIN), so that u = 0 never selects a
 * zero-weight entry; when the prefix sums fall short of u (they end a few
 * ulps below 1), the last entry of positive weight.  torch.multinomial, which
 * the python engine calls (speculative.py:84, :182), never returns a
 * zero-weight index either; its draws are equal in distribution to these. */
static int32_t py_inverse_cdf(const float *x, int64_t V, float u) {
  float cumulative = 0.0f;
  for (int64_t i = 0; i < V; ++i) {
    cumulative += x[i];
    if (cumulative > u && cumulative >= FLT_MIN) return (int32_t)i;
  }
  for (int64_t i = V - 1; i >= 0; --i)
    if (x[i] > 0.0f) return (int32_t)i;
  return (int32_t)(V - 1);
}

int32_t orc_sample_weights(const float *w, int64_t V, float u) {
  float sum = orc_seq_sum(w, V);
  if (!(sum > 0.0f)) return py_inverse_cdf(w, V, u);
  float *x = (float *)malloc((size_t)V * sizeof(float));
  for (int64_t i = 0; i < V; ++i) x[i] = w[i] / sum;
  int32_t t = py_inverse_cdf(x, V, u);
  free(x);
  return t;
}

/* speculative.py:171-182: the weights the resample draws from.  The residual
 * clamp(t - d, 0) divided by its sum (formed sequentially in fp32, as
 * speculative.cpp:30-37 does), or the target row itself when that sum is
 * <= 1e-6.  Returns whether the fallback applied. */
int orc_py_residual_weights(const float *target_p, const float *draft_q,
                            int64_t V, float *out) {
  float sum = 0.0f;
  for (int64_t i = 0; i < V; ++i) {
    out[i] = relu_std_max(target_p[i] - draft_q[i]);
    sum += out[i];
  }
  if (sum <= 1e-6f) {
    for (int64_t i = 0; i < V; ++i) out[i] = target_p[i];
    return 1;
  }
  for (int64_t i = 0; i < V; ++i) out[i] /= sum;
  return 0;
}

/* The python-mode resample: a python-mode inverse-CDF draw from the weights
 * of orc_py_residual_weights. */
int32_t orc_py_sample_adjusted(const float *target_p, const float *draft_q,
                               int64_t V, float u, int *fallback) {
  float *w = (float *)malloc((size_t)V * sizeof(float));
  int fb = orc_py_residual_weights(target_p, draft_q, V, w);
  if (fallback) *fallback = fb;
  int32_t tok = py_inverse_cdf(w, V, u);
  free(w);
  return tok;
}

/* speculative.py:57-84 as the bonus draw sees it: the top-p keep set of the
 * target row, the kept probabilities divided by their sequential fp32 sum
 * (the renormalisation that the softmax over -inf-masked logits performs). */
void orc_py_bonus_weights(const float *pk, int64_t V, float top_p, float *out) {
  uint8_t *keep = (uint8_t *)malloc((size_t)V);
  orc_topp_keep(pk, V, top_p, keep);
  for (int64_t i = 0; i < V; ++i) out[i] = keep[i] ? pk[i] : 0.0f;
  free(keep);
  float sum = orc_seq_sum(out, V);
  if (sum > 0.0f)
    for (int64_t i = 0; i < V; ++i) out[i] /= sum;
}

/* speculative.py:188-195: the top-p filtered bonus draw from target row K.
 * The draw normalises the kept weights by their sequential fp32 sum, exactly
 * as orc_py_bonus_weights does. */
static int32_t py_bonus(const float *pk, int64_t V, float top_p, float u,
                        uint8_t *keep, float *w) {
  orc_topp_keep(pk, V, top_p, keep);
  for (int64_t i = 0; i < V; ++i) w[i] = keep[i] ? pk[i] : 0.0f;
  return orc_sample_weights(w, V, u);
}

/* speculative.py:155-195.  The acceptance test of :161-166 is restated with
 * the fed uniform in place of rand_like: ratio = min(1, q / (p + 1e-8)) in
 * fp32 and accept iff every row has u < ratio.  The resample (:171-182) and
 * the bonus (:188-195) draw with the python-mode inverse CDF on fed uniforms
 * in place of torch.multinomial (equal in distribution, not bit-for-bit).
 * A rejection at the last position (n = K - 1) brings num_accepted to K, so
 * the reference's `num_accepted == self.k` branch (:188) appends the bonus
 * after the resampled token as well. */
int orc_verify_python(int B, int K, int64_t V, int64_t ld, int64_t tsb,
                      int64_t dsb, const float *tprobs, const float *dprobs,
                      const int32_t *tokens, const float *U, float top_p,
                      int32_t *out_n, int32_t *out_num_emitted,
                      int32_t *out_tokens) {
  const int us = K + 2;
  int n = K;
  for (int b = 0; b < B; ++b) {
    int nb = K;
    for (int i = 0; i < K; ++i) {
      int32_t tok = tokens[(int64_t)b * K + i];
      if (tok < 0 || tok >= V) return -2;
      float pd = dprobs[b * dsb + i * ld + tok];
      float qt = tprobs[b * tsb + i * ld + tok];
      float den = pd + 1e-8f;
      float ratio = qt / den;
      if (ratio > 1.0f) ratio = 1.0f;
      if (!(U[(int64_t)b * us + i] < ratio)) {
        nb = i;
        break;
      }
    }
    if (nb < n) n = nb;
  }
  const int extra = (K > 0 && n == K - 1) ? 1 : 0;
  *out_n = n;
  *out_num_emitted = n + 1 + extra;
  uint8_t *keep = (uint8_t *)malloc((size_t)V);
  float *w = (float *)malloc((size_t)V * sizeof(float));
  for (int b = 0; b < B; ++b) {
    int32_t *row = out_tokens + (int64_t)b * (K + 1);
    const float *Ub = U + (int64_t)b * us;
    const float *pk = tprobs + b * tsb + (int64_t)K * ld;
    for (int j = 0; j <= K; ++j) row[j] = -1;
    for (int j = 0; j < n; ++j) row[j] = tokens[(int64_t)b * K + j];
    if (n < K)
      row[n] = orc_py_sample_adjusted(tprobs + b * tsb + n * ld,
                                      dprobs + b * dsb + n * ld, V, Ub[K], NULL);
    else
      row[n] = py_bonus(pk, V, top_p, Ub[K], keep, w);
    if (extra) row[n + 1] = py_bonus(pk, V, top_p, Ub[K + 1], keep, w);
  }
  free(keep);
  free(w);
  return 0;
}

/* ---- tree semantics ---------------------------------------------------- */

/* Residual update after a rejected child: max(0, r - q), sequential fp32 sum,
 * keep r when the sum is <= 1e-6f (the fallback of speculative.cpp:37-40),
 * else divide element-wise (speculative.cpp:43-45). */
static void residual_update(float *r, const float *q, float *tmp, int64_t V) {
  float sum = 0.0f;
  for (int64_t i = 0; i < V; ++i) {
    tmp[i] = relu_std_max(r[i] - q[i]);
    sum += tmp[i];
  }
  if (sum <= 1e-6f) return;
  for (int64_t i = 0; i < V; ++i) r[i] = tmp[i] / sum;
}

int orc_tree_verify(int N, int64_t V, int64_t ld, const int32_t *parent,
                    const int32_t *tok, const float *tprobs,
                    const float *dprobs, int32_t eos, const float *U, int n_u,
                    int greedy, int32_t *out_path, int32_t *out_path_len,
                    int32_t *out_final, int32_t *out_eos, int32_t *out_draws) {
  float *r = (float *)malloc((size_t)V * sizeof(float));
  float *tmp = (float *)malloc((size_t)V * sizeof(float));
  int draws = 0, len = 0, node = 0, rc = 0;
  out_path[len++] = 0;
  *out_eos = 0;
  *out_final = -1;
  for (;;) {
    const float *pn = tprobs + (int64_t)node * ld;
    const float *qn = dprobs + (int64_t)node * ld;
    int first_child = -1;
    for (int c = node + 1; c < N; ++c)
      if (parent[c] == node) {
        first_child = c;
        break;
      }
    if (first_child < 0) { /* leaf: bonus draw from the node's target row */
      if (greedy)
        *out_final = orc_argmax_first(pn, V);
      else {
        if (draws >= n_u) { rc = -1; break; }
        *out_final = orc_sample_from_distribution(pn, V, U[draws++]);
      }
      break;
    }
    int accepted = -1;
    if (greedy) {
      int32_t am = orc_argmax_first(pn, V);
      for (int c = first_child; c < N; ++c)
        if (parent[c] == node && tok[c] == am) {
          accepted = c;
          break;
        }
      if (accepted < 0) {
        *out_final = am;
        break;
      }
    } else {
      memcpy(r, pn, (size_t)V * sizeof(float));
      for (int c = first_child; c < N && accepted < 0; ++c) {
        if (parent[c] != node) continue;
        int32_t x = tok[c];
        float q = qn[x], p = r[x];
        float ratio = (q > 0.0f) ? ((1.0f < p / q) ? 1.0f : p / q) : 0.0f;
        if (draws >= n_u) { rc = -1; break; }
        float u = U[draws++];
        if (u <= ratio)
          accepted = c;
        else
          residual_update(r, qn, tmp, V);
      }
      if (rc) break;
      if (accepted < 0) {
        if (draws >= n_u) { rc = -1; break; }
        *out_final = orc_sample_from_distribution(r, V, U[draws++]);
        break;
      }
    }
    out_path[len++] = accepted;
    node = accepted;
    if (tok[accepted] == eos) {
      *out_final = eos;
      *out_eos = 1;
      break;
    }
  }
  if (*out_final == eos) *out_eos = 1;
  *out_path_len = len;
  *out_draws = draws;
  free(r);
  free(tmp);
  return rc;
}
