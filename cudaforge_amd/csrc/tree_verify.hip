// tree_verify.hip -- acceptance of a draft-token tree: multi-candidate
// rejection sampling down the tree, longest accepted root-to-leaf path, and
// the resample / bonus token, for gfx950.
//
// Tree of N <= 64 nodes, parent[c] < c, node 0 the root (the last verified
// token).  Row n of the target input is the target distribution over the
// token that follows node n; row n of the draft input is the distribution
// node n's children were drawn from.  Walking from the root (cpp semantics of
// csrc/src/scheduler/speculative.cpp:50-103, generalised to several
// candidates per position as in SpecInfer's multi-step speculative sampling):
//   r = p_node
//   for each child c of the node, in increasing index order:
//     x = token[c];  accept iff u <= (q(x) > 0 ? min(1, r(x) / q(x)) : 0)
//     otherwise  r = max(0, r - q) / sum   (sequential fp32 sum; r unchanged
//                when the sum is <= 1e-6, speculative.cpp:26-48)
//   no child accepted:  final = inverse CDF of r (speculative.cpp:11-24)
//   an accepted child becomes the node; an accepted EOS ends the walk
//   a leaf:  final = inverse CDF of p_leaf (the bonus token, :96-97)
// Every test and every final draw consumes the next uniform of the
// sequence's stream.  On a one-child chain this is exactly
// verify_candidates.  Greedy: a child is accepted iff its token is the first
// argmax of p_node; none accepted -> final = that argmax (:105-150).
//
// One 1024-thread work-group per sequence walks its tree.  A visited row's
// softmax statistics (logits input) are computed when the walk first needs
// them, so only visited rows are read; every residual sum and inverse CDF is
// the exact sequential fp32 replay of seqsum.hpp, with the residual chain
// r^(k) = max(0, r^(k-1) - q) / S_k evaluated element-wise on the fly.
#include <hip/hip_runtime.h>

#include <cmath>

#include "abi_internal.hpp"
#include "dist.hpp"
#include "seqsum.hpp"

#pragma clang fp contract(off)

namespace cfa {
namespace treev {

constexpr int kNT = 1024;
constexpr int kMaxN = 64;

struct Args {
  const float *tgt;
  long long t_sb, t_sn;
  const float *drf;
  long long d_sb, d_sn;
  int logits;
  float c;  // log2(e) / temperature
  const int32_t *parent;
  long long parent_sb;
  const int32_t *tok;  // [B, N]
  const float *U;      // [B, n_u]
  int n_u;
  int B, N, V, greedy, eos, vec;
  int32_t *out_path, *out_path_len, *out_tokens, *out_num_emitted, *out_final, *out_eos,
      *out_status;
  float *probs_t, *probs_d;  // optional [B, N, V]: the probabilities of visited rows
};

// r^(k): the residual after k applied normalisations S[0..k).
struct Resid {
  Dist t, d;
  const float *S;
  int k;
  using Raw = float2;
  __device__ __forceinline__ Raw load(long long i) const {
    return make_float2(t.load(i), k > 0 ? d.load(i) : 0.0f);
  }
  __device__ __forceinline__ float eval(Raw v) const {
    float r = t.eval(v.x);
    if (k > 0) {
      const float q = d.eval(v.y);
      for (int j = 0; j < k; ++j) r = relu_ref(r - q) / S[j];
    }
    return r;
  }
};

// max(0, r^(k) - q): the terms of the next residual sum.
struct ResidX {
  Resid r;
  using Raw = float2;
  __device__ __forceinline__ Raw load(long long i) const {
    return make_float2(r.t.load(i), r.d.load(i));
  }
  __device__ __forceinline__ float eval(Raw v) const {
    const float q = r.d.eval(v.y);
    float x = r.t.eval(v.x);
    for (int j = 0; j < r.k; ++j) x = relu_ref(x - q) / r.S[j];
    return relu_ref(x - q);
  }
};

struct __align__(16) Smem {
  seq::Shared<kNT> seq;
  float red_m[kNT / 64], red_s[kNT / 64];
  float Slist[kMaxN];
  int par[kMaxN];
  int tk[kMaxN];
  int path[kMaxN];
  float2 amv[kNT / 64];
  unsigned long long kids;
};

__device__ __forceinline__ const float *trow(const Args &a, int b, int n) {
  return a.tgt + (long long)b * a.t_sb + (long long)n * a.t_sn;
}
__device__ __forceinline__ const float *drow(const Args &a, int b, int n) {
  return a.drf + (long long)b * a.d_sb + (long long)n * a.d_sn;
}

// Softmax statistics (max, 1/sum exp2) of one logits row, block-wide, in a
// fixed reduction order.
__device__ float2 row_stats(const Args &a, const float *row, Smem &sm) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float c = a.c;
  float m = -INFINITY, s = 0.0f;
  // one online update per group of four values: rescale once per new maximum
  auto update = [&](float v0, float v1, float v2, float v3) {
    const float mx = fmaxf(fmaxf(v0, v1), fmaxf(v2, v3));
    if (mx > m) {
      s *= __builtin_amdgcn_exp2f((m - mx) * c);
      m = mx;
    }
    const float ms = (m == -INFINITY) ? 0.0f : m;
    s += __builtin_amdgcn_exp2f((v0 - ms) * c) + __builtin_amdgcn_exp2f((v1 - ms) * c) +
         __builtin_amdgcn_exp2f((v2 - ms) * c) + __builtin_amdgcn_exp2f((v3 - ms) * c);
  };
  if (a.vec) {
    // 16-byte loads, four in flight per thread
    const float4 *p4 = reinterpret_cast<const float4 *>(row);
    const int n4 = a.V / 4;
    constexpr int U = 4;
    int i = tid;
    for (; i + (U - 1) * kNT < n4; i += U * kNT) {
      float4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = p4[i + u * kNT];
#pragma unroll
      for (int u = 0; u < U; ++u) update(v[u].x, v[u].y, v[u].z, v[u].w);
    }
    for (; i < n4; i += kNT) {
      const float4 v = p4[i];
      update(v.x, v.y, v.z, v.w);
    }
  } else {
    for (int i = tid; i < a.V; i += kNT) {
      const float v = row[i];
      if (v > m) {
        s *= __builtin_amdgcn_exp2f((m - v) * c);
        m = v;
      }
      const float ms = (m == -INFINITY) ? 0.0f : m;
      s += __builtin_amdgcn_exp2f((v - ms) * c);
    }
  }
  auto merge = [c](float &m1, float &s1, float m2, float s2) {
    const float M = fmaxf(m1, m2);
    if (M == -INFINITY) return;
    const float f1 = (m1 == M) ? 1.0f : __builtin_amdgcn_exp2f((m1 - M) * c);
    const float f2 = (m2 == M) ? 1.0f : __builtin_amdgcn_exp2f((m2 - M) * c);
    s1 = s1 * f1 + s2 * f2;
    m1 = M;
  };
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float m2 = __shfl_xor(m, d, 64), s2 = __shfl_xor(s, d, 64);
    merge(m, s, m2, s2);
  }
  if (lane == 0) {
    sm.red_m[wave] = m;
    sm.red_s[wave] = s;
  }
  __syncthreads();
  float M = sm.red_m[0], S = sm.red_s[0];
  for (int w = 1; w < kNT / 64; ++w) merge(M, S, sm.red_m[w], sm.red_s[w]);
  __syncthreads();
  return make_float2(M, 1.0f / S);
}

__device__ Dist make_row(const Args &a, const float *row, Smem &sm) {
  Dist d;
  d.p = row;
  d.c = a.c;
  d.logits = a.logits;
  d.M = 0.0f;
  d.invS = 1.0f;
  if (a.logits) {
    const float2 st = row_stats(a, row, sm);
    d.M = st.x;
    d.invS = st.y;
  }
  return d;
}

__device__ void write_probs(const Dist &d, float *dst, int V) {
  if (!dst) return;
  for (int i = threadIdx.x; i < V; i += kNT) dst[i] = d(i);
}

// First index of the largest probability (std::max_element), block-wide.
__device__ int row_argmax(const Dist &d, int V, Smem &sm) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid; i < V; i += kNT) {
    const float v = d(i);
    if (v > bv) {  // strided: indices increase, so ">" keeps the first max
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    const float v2 = __shfl_xor(bv, s, 64);
    const int i2 = __shfl_xor(bi, s, 64);
    if (v2 > bv || (v2 == bv && i2 < bi)) {
      bv = v2;
      bi = i2;
    }
  }
  if (lane == 0) sm.amv[wave] = make_float2(bv, __int_as_float(bi));
  __syncthreads();
  float v = sm.amv[0].x;
  int ix = __float_as_int(sm.amv[0].y);
  for (int w = 1; w < kNT / 64; ++w) {
    const float v2 = sm.amv[w].x;
    const int i2 = __float_as_int(sm.amv[w].y);
    if (v2 > v || (v2 == v && i2 < ix)) {
      v = v2;
      ix = i2;
    }
  }
  __syncthreads();
  return ix == 0x7fffffff ? 0 : ix;
}

__global__ __launch_bounds__(kNT) void tree_verify_kernel(Args a) {
  __shared__ Smem sm;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int N = a.N, V = a.V;
  if (tid < N) {
    sm.par[tid] = a.parent[(long long)b * a.parent_sb + tid];
    sm.tk[tid] = a.tok[(long long)b * N + tid];
  }
  __syncthreads();
  const float *U = a.U ? a.U + (long long)b * a.n_u : nullptr;
  int node = 0, len = 1, draws = 0, fin = -1, eos_acc = 0, status = 0;
  if (tid == 0) sm.path[0] = 0;
  for (;;) {
    // children of `node`, in increasing index order
    unsigned long long kids = 0;
    {
      const bool is_kid = (tid < N) && (tid > node) && sm.par[tid] == node;
      const unsigned long long m = __ballot(is_kid);  // wave 0 holds every node (N <= 64)
      if (tid == 0) sm.kids = m;
      __syncthreads();
      kids = sm.kids;
      __syncthreads();
    }
    const Dist t = make_row(a, trow(a, b, node), sm);
    if (a.probs_t) write_probs(t, a.probs_t + ((long long)b * N + node) * V, V);
    if (!kids) {  // a leaf: the bonus token
      if (a.greedy) {
        fin = row_argmax(t, V, sm);
      } else {
        if (draws >= a.n_u) {
          status = 1;
          break;
        }
        long long idx = -1;
        seq::run<kNT>(Resid{t, t, sm.Slist, 0}, V, true, U[draws++], sm.seq, &idx);
        fin = (idx < 0) ? V - 1 : (int)idx;
      }
      break;
    }
    int accepted = -1;
    if (a.greedy) {
      const int am = row_argmax(t, V, sm);
      for (unsigned long long m = kids; m; m &= m - 1) {
        const int c = __builtin_ctzll(m);
        if (sm.tk[c] == am) {
          accepted = c;
          break;
        }
      }
      if (accepted < 0) {
        fin = am;
        break;
      }
    } else {
      const Dist d = make_row(a, drow(a, b, node), sm);
      if (a.probs_d) write_probs(d, a.probs_d + ((long long)b * N + node) * V, V);
      int k = 0;  // applied normalisations of the residual
      for (unsigned long long m = kids; m; m &= m - 1) {
        const int c = __builtin_ctzll(m);
        const int x = sm.tk[c];
        const bool valid = x >= 0 && x < V;
        const int xs = valid ? x : 0;
        const Resid r{t, d, sm.Slist, k};
        const float p = r.eval(r.load(xs));  // r^(k)(x)
        const float q = d(xs);
        const float ratio = valid ? ratio_cpp(p, q) : -1.0f;  // an out-of-range id never passes
        if (draws >= a.n_u) {
          status = 1;
          break;
        }
        const float u = U[draws++];
        if (u <= ratio) {
          accepted = c;
          break;
        }
        const float S = seq::run<kNT>(ResidX{r}, V, false, 0.0f, sm.seq, nullptr);
        if (S > 1e-6f) {  // else the residual stays (speculative.cpp:37-40)
          if (tid == 0) sm.Slist[k] = S;
          __syncthreads();
          ++k;
        }
      }
      if (status) break;
      if (accepted < 0) {
        if (draws >= a.n_u) {
          status = 1;
          break;
        }
        long long idx = -1;
        seq::run<kNT>(Resid{t, d, sm.Slist, k}, V, true, U[draws++], sm.seq, &idx);
        fin = (idx < 0) ? V - 1 : (int)idx;
        break;
      }
    }
    if (tid == 0) sm.path[len] = accepted;
    ++len;
    node = accepted;
    if (sm.tk[accepted] == a.eos) {
      fin = a.eos;
      eos_acc = 1;
      break;
    }
  }
  __syncthreads();
  // outputs: path (root first), emitted tokens (accepted drafts then final)
  const long long ob = (long long)b * N;
  for (int j = tid; j < N; j += kNT) a.out_path[ob + j] = (j < len) ? sm.path[j] : -1;
  for (int j = tid; j <= N; j += kNT) {
    int v = -1;
    if (j < len - 1) v = sm.tk[sm.path[j + 1]];
    if (j == len - 1 && !eos_acc && !status) v = fin;
    a.out_tokens[(long long)b * (N + 1) + j] = v;
  }
  if (tid == 0) {
    a.out_path_len[b] = len;
    a.out_final[b] = status ? -1 : fin;
    a.out_eos[b] = (!status && (eos_acc || fin == a.eos)) ? 1 : 0;
    a.out_num_emitted[b] = status ? len - 1 : (eos_acc ? len - 1 : len);
    if (a.out_status) a.out_status[b] = status;
  }
}

}  // namespace treev
}  // namespace cfa

using namespace cfa;

extern "C" int cfa_tree_verify(const float *target, int64_t t_stride_b, int64_t t_stride_n,
                               const float *draft, int64_t d_stride_b, int64_t d_stride_n,
                               int input_kind, const int32_t *parents, int64_t parents_stride_b,
                               const int32_t *node_tokens, const float *uniforms, int n_uniforms,
                               int B, int N, int V, float temperature, int mode,
                               int32_t eos_token_id, int32_t *out_path, int32_t *out_path_len,
                               int32_t *out_tokens, int32_t *out_num_emitted, int32_t *out_final,
                               int32_t *out_eos, int32_t *out_status, float *out_target_probs,
                               float *out_draft_probs, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (B <= 0 || N <= 0 || N > treev::kMaxN || V <= 0)
    return fail_arg("need B > 0, 0 < N <= 64 and V > 0");
  if (mode != CFA_MODE_CPP && mode != CFA_MODE_GREEDY)
    return fail_arg("tree verification supports CFA_MODE_CPP and CFA_MODE_GREEDY");
  if (input_kind != CFA_INPUT_PROBS && input_kind != CFA_INPUT_LOGITS)
    return fail_arg("input_kind must be CFA_INPUT_PROBS or CFA_INPUT_LOGITS");
  const bool greedy = mode == CFA_MODE_GREEDY;
  if (!target || !parents || !node_tokens || (!greedy && (!draft || !uniforms || n_uniforms < 1)))
    return fail_arg("null input pointer");
  if (!out_path || !out_path_len || !out_tokens || !out_num_emitted || !out_final || !out_eos)
    return fail_arg("null output pointer");
  if (input_kind == CFA_INPUT_LOGITS && !(temperature > 0.0f)) return fail_arg("temperature must be > 0");
  if (t_stride_n < V || t_stride_b < (int64_t)N * t_stride_n) return fail_arg("target strides overlap rows");
  if (!greedy && (d_stride_n < V || d_stride_b < (int64_t)N * d_stride_n))
    return fail_arg("draft strides overlap rows");
  if (B > 2147483647 / 2) return fail_arg("B too large");
  treev::Args a{};
  a.tgt = target;
  a.t_sb = t_stride_b;
  a.t_sn = t_stride_n;
  a.drf = draft;
  a.d_sb = d_stride_b;
  a.d_sn = d_stride_n;
  a.logits = input_kind == CFA_INPUT_LOGITS;
  a.c = a.logits ? (float)(1.4426950408889634 / (double)temperature) : 1.0f;
  a.parent = parents;
  a.parent_sb = parents_stride_b;
  a.tok = node_tokens;
  a.U = uniforms;
  a.n_u = greedy ? 0 : n_uniforms;
  a.B = B;
  a.N = N;
  a.V = V;
  a.greedy = greedy ? 1 : 0;
  a.eos = eos_token_id;
  a.out_path = out_path;
  a.out_path_len = out_path_len;
  a.out_tokens = out_tokens;
  a.out_num_emitted = out_num_emitted;
  a.out_final = out_final;
  a.out_eos = out_eos;
  a.out_status = out_status;
  a.probs_t = out_target_probs;
  a.probs_d = greedy ? nullptr : out_draft_probs;
  // 16-byte vector loads need every row 16-byte aligned
  a.vec = (V % 4 == 0) && (t_stride_b % 4 == 0) && (t_stride_n % 4 == 0) &&
          (((uintptr_t)target & 15) == 0) &&
          (greedy || ((d_stride_b % 4 == 0) && (d_stride_n % 4 == 0) && (((uintptr_t)draft & 15) == 0)));
  CFA_LAUNCH("tree_verify", treev::tree_verify_kernel, dim3(B), dim3(treev::kNT), 0,
             (hipStream_t)stream, a);
  return CFA_OK;
}
