// chain_verify.hip -- batched chain verification for gfx950.
//
// One call verifies B sequences of K draft tokens against the target model:
//   stats   : one streaming pass over the target [B,K+1,V] and draft [B,K,V]
//             logits -> per-row (max, sum exp) partials (logits input only);
//   decide  : one wave per sequence gathers p/q at the draft tokens and runs
//             the acceptance walk (speculative.cpp:66-97 or
//             speculative.py:155-185), leaving at most one draw per row;
//   sample  : one work-group per sequence performs that draw with the exact
//             sequential-fp32 inverse CDF of speculative.cpp:11-48
//             (seqsum.hpp), then writes the outputs.
// Greedy mode (speculative.cpp:105-150) replaces sample by a first-argmax pass.
//
// Probabilities computed from logits (the fused path) are
//   p_i = exp2((l_i - max_l) * c) * (1 / S),  c = log2(e) / T,
//   S   = sum_j exp2((l_j - max_l) * c),
// evaluated identically everywhere they are used, so the decisions equal the
// oracle's when the oracle is fed these p_i (optionally written out).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "abi_internal.hpp"
#include "seqsum.hpp"

// Every fp32 expression below must round exactly as written (the oracle and
// the reference evaluate t_i - d_i, p / q and x / S as separate roundings).
#pragma clang fp contract(off)

namespace cfa {
namespace chain {

enum Kind : int { kNone = 0, kResid = 1, kPlain = 2, kPyBonus = 3 };

struct Args {
  const float *tgt;
  long long t_sb, t_sk;
  const float *drf;
  long long d_sb, d_sk;
  const int32_t *tokens;  // [B,K]
  const float *U;         // [B,K+1]
  int B, K, V, rpb;       // rows per sequence: K+1 (greedy) or 2K+1
  float c;                // log2(e) / temperature
  int logits;             // 1: inputs are logits
  int mode;               // CFA_MODE_*
  int eos;
  float top_p;
  // partition of the stats / argmax passes
  long long Vw;  // row length in vector units
  long long C;   // units per work-group
  int G;         // work-groups
  float2 *part;  // [G*2] (max logit, sum exp) per (wg, row slot)
  float2 *apart; // [G*2] (max prob, index as bits) per (wg, row slot)
  int4 *dec;     // [B] {n_b, kind, row, eos_accepted}
  float *ufin;   // [B]
  int32_t *out_accept_len, *out_tokens, *out_num_emitted, *out_final, *out_eos;
};

__device__ __forceinline__ const float *row_ptr(const Args &a, int b, int j) {
  return j <= a.K ? a.tgt + (long long)b * a.t_sb + (long long)j * a.t_sk
                  : a.drf + (long long)b * a.d_sb + (long long)(j - a.K - 1) * a.d_sk;
}

// A row's probabilities: stored probs, or logits with (max, 1/S).  load()
// only reads memory and eval() does the arithmetic, so seq::run can keep the
// next block's loads in flight while it sweeps the current one.
struct Dist {
  const float *p;
  float M, invS, c;
  int logits;
  using Raw = float;
  __device__ __forceinline__ Raw load(long long i) const { return p[i]; }
  __device__ __forceinline__ float eval(Raw v) const {
    return logits ? __builtin_amdgcn_exp2f((v - M) * c) * invS : v;
  }
  __device__ __forceinline__ float operator()(long long i) const { return eval(load(i)); }
};

// (max, 1/S) of row r from the stats partials, combined in a fixed order.
__device__ float2 row_stat(const Args &a, int r) {
  const long long lo = (long long)r * a.Vw, hi = lo + a.Vw - 1;
  const long long w0 = lo / a.C, w1 = hi / a.C;
  float M = -INFINITY;
  for (long long w = w0; w <= w1; ++w) {
    const int slot = r - (int)((w * a.C) / a.Vw);
    M = fmaxf(M, a.part[2 * w + slot].x);
  }
  float S = 0.0f;
  for (long long w = w0; w <= w1; ++w) {
    const int slot = r - (int)((w * a.C) / a.Vw);
    const float2 ms = a.part[2 * w + slot];
    S += (ms.x == M) ? ms.y : ms.y * __builtin_amdgcn_exp2f((ms.x - M) * a.c);
  }
  return make_float2(M, 1.0f / S);
}

__device__ Dist make_dist(const Args &a, int b, int j) {
  Dist d;
  d.p = row_ptr(a, b, j);
  d.c = a.c;
  d.logits = a.logits;
  d.M = 0.0f;
  d.invS = 1.0f;
  if (a.logits) {
    const float2 st = row_stat(a, b * a.rpb + j);
    d.M = st.x;
    d.invS = st.y;
  }
  return d;
}

// ---------------------------------------------------------------------------
// stats: online (max, sum exp2) over a balanced slice of the row space.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void ms_merge(float &m, float &s, float m2, float s2, float c) {
  const float M = fmaxf(m, m2);
  if (M == -INFINITY) return;
  const float f1 = (m == M) ? 1.0f : __builtin_amdgcn_exp2f((m - M) * c);
  const float f2 = (m2 == M) ? 1.0f : __builtin_amdgcn_exp2f((m2 - M) * c);
  s = s * f1 + s2 * f2;
  m = M;
}

template <int NT>
__device__ float2 block_ms(float m, float s, float c) {
  __shared__ float2 red[NT / 64];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float m2 = __shfl_xor(m, d, 64);
    const float s2 = __shfl_xor(s, d, 64);
    ms_merge(m, s, m2, s2, c);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = make_float2(m, s);
  __syncthreads();
  float2 out = red[0];
  for (int w = 1; w < NT / 64; ++w) ms_merge(out.x, out.y, red[w].x, red[w].y, c);
  __syncthreads();
  return out;
}

template <int NT, int W>
__global__ __launch_bounds__(NT) void stats_kernel(Args a) {
  const long long total = (long long)a.B * a.rpb * a.Vw;
  const long long lo = (long long)blockIdx.x * a.C;
  const long long hi = min(lo + a.C, total);
  if (lo >= hi) return;
  const float c = a.c;
  int slot = 0;
  for (long long r = lo / a.Vw; r * a.Vw < hi; ++r, ++slot) {
    const long long s0 = max(lo, r * a.Vw) - r * a.Vw;
    const long long s1 = min(hi, (r + 1) * a.Vw) - r * a.Vw;
    const float *row = row_ptr(a, (int)(r / a.rpb), (int)(r % a.rpb));
    float m = -INFINITY, s = 0.0f;
    if (W == 4) {
      const float4 *p4 = reinterpret_cast<const float4 *>(row);
      long long i = s0 + threadIdx.x;
      constexpr int U = 8;
      for (; i + (U - 1) * NT < s1; i += U * NT) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = p4[i + u * NT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float mx = fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w));
          if (mx > m) {
            s *= __builtin_amdgcn_exp2f((m - mx) * c);
            m = mx;
          }
          const float ms = (m == -INFINITY) ? 0.0f : m;
          s += __builtin_amdgcn_exp2f((v[u].x - ms) * c) + __builtin_amdgcn_exp2f((v[u].y - ms) * c) +
               __builtin_amdgcn_exp2f((v[u].z - ms) * c) + __builtin_amdgcn_exp2f((v[u].w - ms) * c);
        }
      }
      for (; i < s1; i += NT) {
        const float4 v = p4[i];
        const float mx = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
        if (mx > m) {
          s *= __builtin_amdgcn_exp2f((m - mx) * c);
          m = mx;
        }
        const float ms = (m == -INFINITY) ? 0.0f : m;
        s += __builtin_amdgcn_exp2f((v.x - ms) * c) + __builtin_amdgcn_exp2f((v.y - ms) * c) +
             __builtin_amdgcn_exp2f((v.z - ms) * c) + __builtin_amdgcn_exp2f((v.w - ms) * c);
      }
    } else {
      for (long long i = s0 + threadIdx.x; i < s1; i += NT) {
        const float v = row[i];
        if (v > m) {
          s *= __builtin_amdgcn_exp2f((m - v) * c);
          m = v;
        }
        const float ms = (m == -INFINITY) ? 0.0f : m;
        s += __builtin_amdgcn_exp2f((v - ms) * c);
      }
    }
    const float2 out = block_ms<NT>(m, s, c);
    if (threadIdx.x == 0) a.part[2 * blockIdx.x + slot] = out;
  }
}

// ---------------------------------------------------------------------------
// argmax (greedy): first index of the largest probability of target rows.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void am_merge(float &v, int &i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

template <int NT>
__global__ __launch_bounds__(NT) void argmax_kernel(Args a) {
  const long long total = (long long)a.B * a.rpb * a.Vw;
  const long long lo = (long long)blockIdx.x * a.C;
  const long long hi = min(lo + a.C, total);
  if (lo >= hi) return;
  __shared__ float2 red[NT / 64];
  const int W = (int)(a.V / a.Vw);
  int slot = 0;
  for (long long r = lo / a.Vw; r * a.Vw < hi; ++r, ++slot) {
    const long long e0 = (max(lo, r * a.Vw) - r * a.Vw) * W;
    const long long e1 = (min(hi, (r + 1) * a.Vw) - r * a.Vw) * W;
    const Dist d = make_dist(a, (int)(r / a.rpb), (int)(r % a.rpb));
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (long long i = e0 + threadIdx.x; i < e1; i += NT) am_merge(bv, bi, d(i), (int)i);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
      const float v2 = __shfl_xor(bv, s, 64);
      const int i2 = __shfl_xor(bi, s, 64);
      am_merge(bv, bi, v2, i2);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = make_float2(bv, __int_as_float(bi));
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = red[0].x;
      int ix = __float_as_int(red[0].y);
      for (int w = 1; w < NT / 64; ++w) am_merge(v, ix, red[w].x, __float_as_int(red[w].y));
      a.apart[2 * blockIdx.x + slot] = make_float2(v, __int_as_float(ix));
    }
    __syncthreads();
  }
}

__device__ int row_argmax(const Args &a, int r) {
  const long long lo = (long long)r * a.Vw, hi = lo + a.Vw - 1;
  float v = -INFINITY;
  int ix = 0x7fffffff;
  for (long long w = lo / a.C; w <= hi / a.C; ++w) {
    const int slot = r - (int)((w * a.C) / a.Vw);
    const float2 e = a.apart[2 * w + slot];
    am_merge(v, ix, e.x, __float_as_int(e.y));
  }
  return ix == 0x7fffffff ? 0 : ix;
}

// ---------------------------------------------------------------------------
// decide: one wave per sequence.
// ---------------------------------------------------------------------------

constexpr int kMaxK = 64;

__global__ __launch_bounds__(64) void decide_kernel(Args a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  __shared__ float pt[kMaxK], qd[kMaxK];
  __shared__ int tk[kMaxK], am[kMaxK + 1], ok[kMaxK];
  const int K = a.K;
  for (int i = lane; i < K; i += 64) {
    int t = a.tokens[(long long)b * K + i];
    tk[i] = t;
    t = min(max(t, 0), a.V - 1);  // never read outside the row
    if (a.mode != CFA_MODE_GREEDY) {
      const bool valid = (a.tokens[(long long)b * K + i] == t);
      const Dist dt = make_dist(a, b, i);
      const Dist dd = make_dist(a, b, K + 1 + i);
      pt[i] = valid ? dt(t) : 0.0f;
      qd[i] = valid ? dd(t) : 0.0f;
      ok[i] = valid ? 1 : 0;  // an id outside [0, V) is never accepted
    }
  }
  if (a.mode == CFA_MODE_GREEDY)
    for (int i = lane; i <= K; i += 64) am[i] = row_argmax(a, b * a.rpb + i);
  __syncthreads();
  if (lane != 0) return;
  const float *U = a.U + (long long)b * (K + 1);
  int n = 0, kind = kNone, row = -1, eos_acc = 0;
  float uf = 0.0f;
  if (a.mode == CFA_MODE_CPP) {
    int draws = 0;
    for (int i = 0; i < K; ++i) {
      const float ratio = ratio_cpp(pt[i], qd[i]);
      const float r = U[draws++];
      if (ok[i] && r <= ratio) {
        ++n;
        if (tk[i] == a.eos) {
          eos_acc = 1;
          break;
        }
      } else {
        kind = kResid;
        row = i;
        uf = U[draws++];
        break;
      }
    }
    if (!eos_acc && kind == kNone) {
      kind = kPlain;
      row = K;
      uf = U[draws++];
    }
  } else if (a.mode == CFA_MODE_PYTHON) {
    n = K;
    for (int i = 0; i < K; ++i)
      if (!(U[i] < ratio_py(pt[i], qd[i]))) {
        n = i;
        break;
      }
    uf = U[K];
  } else {  // greedy: outputs are final here
    int fin = -1;
    for (int i = 0; i < K; ++i) {
      if (tk[i] == am[i]) {
        ++n;
        if (tk[i] == a.eos) {
          eos_acc = 1;
          fin = a.eos;
          break;
        }
      } else {
        fin = am[i];
        break;
      }
    }
    if (!eos_acc && n == K) fin = am[K];
    int32_t *ot = a.out_tokens + (long long)b * (K + 1);
    for (int j = 0; j <= K; ++j) ot[j] = (j < n) ? tk[j] : -1;
    if (!eos_acc) ot[n] = fin;
    a.out_accept_len[b] = n;
    a.out_final[b] = fin;
    a.out_eos[b] = (eos_acc || fin == a.eos) ? 1 : 0;
    a.out_num_emitted[b] = eos_acc ? n : n + 1;
    return;
  }
  a.dec[b] = make_int4(n, kind, row, eos_acc);
  a.ufin[b] = uf;
}

// ---------------------------------------------------------------------------
// sample: one work-group per sequence, exact sequential inverse CDF.
// ---------------------------------------------------------------------------

struct XResid {  // max(0, t_i - d_i)            (speculative.cpp:33)
  Dist t, d;
  using Raw = float2;
  __device__ __forceinline__ Raw load(long long i) const { return make_float2(t.load(i), d.load(i)); }
  __device__ __forceinline__ float eval(Raw v) const { return relu_ref(t.eval(v.x) - d.eval(v.y)); }
};
struct XResidNorm {  // max(0, t_i - d_i) / sum    (speculative.cpp:44)
  Dist t, d;
  float S;
  using Raw = float2;
  __device__ __forceinline__ Raw load(long long i) const { return make_float2(t.load(i), d.load(i)); }
  __device__ __forceinline__ float eval(Raw v) const {
    return relu_ref(t.eval(v.x) - d.eval(v.y)) / S;
  }
};
struct XKeep {  // top-p kept probabilities (speculative.py:67-83)
  Dist t;
  float vstar;
  using Raw = float;
  __device__ __forceinline__ Raw load(long long i) const { return t.load(i); }
  __device__ __forceinline__ float eval(Raw v) const {
    const float p = t.eval(v);
    return (p >= vstar) ? p : 0.0f;
  }
};
struct XKeepNorm {
  Dist t;
  float vstar, S;
  using Raw = float;
  __device__ __forceinline__ Raw load(long long i) const { return t.load(i); }
  __device__ __forceinline__ float eval(Raw v) const {
    const float p = t.eval(v);
    return ((p >= vstar) ? p : 0.0f) / S;
  }
};

template <int NT>
__device__ double block_sum_f64(double v, double *red) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < NT / 64; ++w) t += red[w];
  return t;
}

// Smallest kept probability of the top-p rule: the least v with
// sum_{p_i > v} p_i <= top_p (fp64), found by bisection on the fp32 bits.
template <int NT>
__device__ float topp_threshold(const Dist &t, int V, float top_p, double *red) {
  uint32_t lo = 0, hi = 0x7f800000u;
  while (hi - lo > 1) {
    const uint32_t mid = lo + (hi - lo) / 2;
    const float tau = u2f(mid);
    double acc = 0.0;
    for (int i = threadIdx.x; i < V; i += NT) {
      const float p = t(i);
      if (p > tau) acc += (double)p;
    }
    const double F = block_sum_f64<NT>(acc, red);
    if (F <= (double)top_p)
      hi = mid;
    else
      lo = mid;
  }
  return u2f(hi);
}

constexpr int kSampleNT = 1024;

__global__ __launch_bounds__(kSampleNT) void sample_kernel(Args a) {
  __shared__ seq::Shared<kSampleNT> sh;
  __shared__ double red[kSampleNT / 64];
  __shared__ int nmin;
  const int b = blockIdx.x, K = a.K, V = a.V;
  int4 dj = a.dec[b];
  int n = dj.x, kind = dj.y, row = dj.z;
  const int eos_acc = dj.w;
  const float u = a.ufin[b];
  if (a.mode == CFA_MODE_PYTHON) {  // batch lock-step: n = min_b n_b (speculative.py:166)
    if (threadIdx.x == 0) nmin = K;
    __syncthreads();
    int local = K;
    for (int q = threadIdx.x; q < a.B; q += kSampleNT) local = min(local, a.dec[q].x);
    atomicMin(&nmin, local);
    __syncthreads();
    n = nmin;
    kind = (n < K) ? kResid : kPyBonus;
    row = (n < K) ? n : K;
  }
  int fin = -1;
  if (kind != kNone) {
    const Dist t = make_dist(a, b, row);
    long long idx = -1;
    if (kind == kResid) {
      const Dist d = make_dist(a, b, K + 1 + row);
      const float S = seq::run<kSampleNT>(XResid{t, d}, V, false, 0.0f, sh, nullptr);
      if (S <= 1e-6f)
        seq::run<kSampleNT>(t, V, true, u, sh, &idx);  // speculative.cpp:37-40
      else
        seq::run<kSampleNT>(XResidNorm{t, d, S}, V, true, u, sh, &idx);
    } else if (kind == kPlain) {
      seq::run<kSampleNT>(t, V, true, u, sh, &idx);  // speculative.cpp:97
    } else {  // python bonus: top-p filter, renormalise, draw
      const float vstar = (a.top_p < 1.0f) ? topp_threshold<kSampleNT>(t, V, a.top_p, red) : 0.0f;
      const float S = seq::run<kSampleNT>(XKeep{t, vstar}, V, false, 0.0f, sh, nullptr);
      if (S > 0.0f)
        seq::run<kSampleNT>(XKeepNorm{t, vstar, S}, V, true, u, sh, &idx);
      else
        seq::run<kSampleNT>(XKeep{t, vstar}, V, true, u, sh, &idx);
    }
    fin = (idx < 0) ? V - 1 : (int)idx;
  }
  if (threadIdx.x <= K) {
    const int j = threadIdx.x;
    int v = -1;
    if (j < n) v = a.tokens[(long long)b * K + j];
    if (j == n && !eos_acc) v = fin;
    a.out_tokens[(long long)b * (K + 1) + j] = v;
  }
  if (threadIdx.x == 0) {
    if (eos_acc) fin = a.eos;
    a.out_accept_len[b] = n;
    a.out_final[b] = fin;
    a.out_eos[b] = (a.mode == CFA_MODE_CPP) ? ((eos_acc || fin == a.eos) ? 1 : 0) : 0;
    a.out_num_emitted[b] = eos_acc ? n : n + 1;
  }
}

// Optional: write the probabilities the verification used.
__global__ __launch_bounds__(256) void probs_out_kernel(Args a, float *out_t, float *out_d) {
  const int r = blockIdx.y;
  const int b = r / a.rpb, j = r % a.rpb;
  float *dst = (j <= a.K) ? out_t + ((long long)b * (a.K + 1) + j) * a.V
                          : out_d + ((long long)b * a.K + (j - a.K - 1)) * a.V;
  if ((j <= a.K && !out_t) || (j > a.K && !out_d)) return;
  const Dist d = make_dist(a, b, j);
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < a.V; i += (long long)gridDim.x * 256)
    dst[i] = d(i);
}

}  // namespace chain
}  // namespace cfa

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
using namespace cfa;
using namespace cfa::chain;

static size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

static int max_groups(int R) { return std::max(R, 8192); }

extern "C" size_t cfa_chain_verify_workspace_size(int B, int K, int V, int input_kind, int mode) {
  (void)V;
  (void)input_kind;
  if (B <= 0 || K < 0) return 0;
  const int rpb = (mode == CFA_MODE_GREEDY) ? K + 1 : 2 * K + 1;
  const size_t G = (size_t)max_groups(B * rpb);
  return align_up(G * 2 * sizeof(float2)) * 2 + align_up((size_t)B * sizeof(int4)) +
         align_up((size_t)B * sizeof(float));
}

extern "C" int cfa_chain_verify(const float *target, int64_t t_stride_b, int64_t t_stride_k,
                                const float *draft, int64_t d_stride_b, int64_t d_stride_k,
                                int input_kind, const int32_t *draft_tokens, const float *uniforms,
                                int B, int K, int V, float temperature, float top_p, int mode,
                                int32_t eos_token_id, int32_t *out_accept_len, int32_t *out_tokens,
                                int32_t *out_num_emitted, int32_t *out_final, int32_t *out_eos,
                                float *out_target_probs, float *out_draft_probs, void *workspace,
                                size_t workspace_bytes, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (B <= 0 || K < 0 || V <= 0) return fail_arg("B and V must be positive and K >= 0");
  if (K > kMaxK - 1) return fail_arg("K must be at most 63");
  if (mode != CFA_MODE_CPP && mode != CFA_MODE_PYTHON && mode != CFA_MODE_GREEDY)
    return fail_arg("mode must be CFA_MODE_CPP, CFA_MODE_PYTHON or CFA_MODE_GREEDY");
  if (input_kind != CFA_INPUT_PROBS && input_kind != CFA_INPUT_LOGITS)
    return fail_arg("input_kind must be CFA_INPUT_PROBS or CFA_INPUT_LOGITS");
  if (!target || (K > 0 && !draft_tokens)) return fail_arg("null input pointer");
  if (mode != CFA_MODE_GREEDY && ((K > 0 && !draft) || !uniforms)) return fail_arg("null input pointer");
  if (!out_accept_len || !out_tokens || !out_num_emitted || !out_final || !out_eos)
    return fail_arg("null output pointer");
  if (input_kind == CFA_INPUT_LOGITS && !(temperature > 0.0f)) return fail_arg("temperature must be > 0");
  if (t_stride_k < V || t_stride_b < (int64_t)(K + 1) * t_stride_k)
    return fail_arg("target strides overlap rows");
  if (K > 0 && mode != CFA_MODE_GREEDY && (d_stride_k < V || d_stride_b < (int64_t)K * d_stride_k))
    return fail_arg("draft strides overlap rows");
  const size_t need = cfa_chain_verify_workspace_size(B, K, V, input_kind, mode);
  if (!workspace || workspace_bytes < need) return fail_arg("workspace too small (see cfa_chain_verify_workspace_size)");

  Args a{};
  a.tgt = target;
  a.t_sb = t_stride_b;
  a.t_sk = t_stride_k;
  a.drf = draft;
  a.d_sb = d_stride_b;
  a.d_sk = d_stride_k;
  a.tokens = draft_tokens;
  a.U = uniforms;
  a.B = B;
  a.K = K;
  a.V = V;
  a.rpb = (mode == CFA_MODE_GREEDY) ? K + 1 : 2 * K + 1;
  a.logits = input_kind == CFA_INPUT_LOGITS;
  a.c = a.logits ? (float)(1.4426950408889634 / (double)temperature) : 1.0f;
  a.mode = mode;
  a.eos = eos_token_id;
  a.top_p = top_p;
  a.out_accept_len = out_accept_len;
  a.out_tokens = out_tokens;
  a.out_num_emitted = out_num_emitted;
  a.out_final = out_final;
  a.out_eos = out_eos;

  // vector loads need 16-byte aligned rows
  const bool vec = (V % 4 == 0) && (t_stride_k % 4 == 0) && (t_stride_b % 4 == 0) &&
                   (((uintptr_t)target & 15) == 0) &&
                   (mode == CFA_MODE_GREEDY || K == 0 ||
                    ((d_stride_k % 4 == 0) && (d_stride_b % 4 == 0) && (((uintptr_t)draft & 15) == 0)));
  const int W = vec ? 4 : 1;
  a.Vw = V / W;
  const int R = B * a.rpb;
  const long long total = (long long)R * a.Vw;
  const int cus = device_cu_count();
  long long G = std::min<long long>((long long)cus * 8, (total + 1023) / 1024);
  G = std::max<long long>(G, R);
  G = std::min<long long>(G, max_groups(R));
  a.C = (total + G - 1) / G;
  a.G = (int)((total + a.C - 1) / a.C);

  char *ws = (char *)workspace;
  const size_t Gmax = (size_t)max_groups(R);
  a.part = (float2 *)ws;
  ws += align_up(Gmax * 2 * sizeof(float2));
  a.apart = (float2 *)ws;
  ws += align_up(Gmax * 2 * sizeof(float2));
  a.dec = (int4 *)ws;
  ws += align_up((size_t)B * sizeof(int4));
  a.ufin = (float *)ws;

  hipStream_t st = (hipStream_t)stream;
  if (a.logits) {
    if (vec)
      CFA_LAUNCH("chain_stats", (stats_kernel<256, 4>), dim3(a.G), dim3(256), 0, st, a);
    else
      CFA_LAUNCH("chain_stats", (stats_kernel<256, 1>), dim3(a.G), dim3(256), 0, st, a);
  }
  if (mode == CFA_MODE_GREEDY)
    CFA_LAUNCH("chain_argmax", (argmax_kernel<256>), dim3(a.G), dim3(256), 0, st, a);
  CFA_LAUNCH("chain_decide", decide_kernel, dim3(B), dim3(64), 0, st, a);
  if (mode != CFA_MODE_GREEDY)
    CFA_LAUNCH("chain_sample", sample_kernel, dim3(B), dim3(kSampleNT), 0, st, a);
  if (out_target_probs || out_draft_probs) {
    const int rows = B * a.rpb;
    const int gx = std::min(64, (V + 255) / 256);
    CFA_LAUNCH("chain_probs_out", probs_out_kernel, dim3(gx, rows), dim3(256), 0, st, a,
               out_target_probs, out_draft_probs);
  }
  return CFA_OK;
}
