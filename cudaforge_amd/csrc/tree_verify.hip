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
// A team of G <= 8 work-groups per sequence (team.hpp) walks its tree: each visited row's softmax statistics (logits input) are
// reduced over the team, each member reading its slice of the row, so only
// visited rows are read; every residual sum and inverse CDF is the exact
// sequential fp32 replay of seqsum.hpp split over the team (team_seq), with
// the residual chain r^(k) = max(0, r^(k-1) - q) / S_k evaluated element-wise
// on the fly.  With more sequences than teams, each team walks several.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>

#include "abi_internal.hpp"
#include "dist.hpp"
#include "lds_dma.hpp"
#include "seqsum.hpp"
#include "team.hpp"

#pragma clang fp contract(off)

namespace cfa {
namespace treev {

constexpr int kNT = 1024;
constexpr int kMaxN = 64;
constexpr int kMaxU = 256;  // uniforms staged in LDS per sequence

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
  int T, G;              // teams, work-groups per team
  team::State *teams;    // [T] (zero before the launch)
  int *err;              // team wait timed out somewhere
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

// fp32 bounds on a double: the largest float <= v and the smallest >= v.
__device__ __forceinline__ float f32_down(double v) {
  float f = (float)v;
  if ((double)f > v) f = __uint_as_float(__float_as_uint(f) - 1u);  // v > 0 here
  return f;
}
__device__ __forceinline__ float f32_up(double v) {
  float f = (float)v;
  if ((double)f < v) f = __uint_as_float(__float_as_uint(f) + 1u);
  return f;
}

// Early exit of the residual sum S = sum max(0, r^(k) - q) that a rejected
// child needs only for its next sibling's test: given the blocked fp32 total
// Sb of the same terms (at most `depth` additions deep), the sequential sum
// lies in [Sb (1 - g_n) / (1 + g_depth), Sb (1 + g_n) / (1 - g_depth)] with
// g_k = k u / (1 - k u), u = 2^-24 (the standard bound for sums of
// non-negative terms).  The sibling's ratio min(1, r^(k+1)(x) / q(x)),
// r^(k+1)(x) = max(0, r^(k)(x) - q(x)) / S, does not increase with S, so if
// its uniform passes at the largest S (and the <= 1e-6 fallback is excluded)
// it is accepted whatever the exact S is: the exact walk is skipped.
// (A handful of scalars, passed by value: a larger functor would be passed
// through scratch memory.)
struct SiblingAccepts {
  float p;  // r^(k) at the sibling's token
  float q;  // the draft probability there
  float u;  // its uniform
  long long n;
  __device__ SiblingAccepts(const Resid &r, float2 raw, float u_, long long n_)
      : p(r.eval(raw)), q(r.d.eval(raw.y)), u(u_), n(n_) {}
  __device__ bool operator()(float Sb, int depth) const {
    const double u24 = 5.9604644775390625e-08;
    const double gn = (double)n * u24 / (1.0 - (double)n * u24);
    const double gd = (double)depth * u24 / (1.0 - (double)depth * u24);
    if (!(gn < 0.5) || !(gd < 0.5)) return false;
    const float lo = f32_down((double)Sb * (1.0 - gn) / (1.0 + gd));
    const float hi = f32_up((double)Sb * (1.0 + gn) / (1.0 - gd));
    if (!(lo > 1e-6f) || !(hi < INFINITY)) return false;
    const float ratio = ratio_cpp(relu_ref(p - q) / hi, q);
    return u <= ratio;
  }
};

struct __align__(16) Smem {
  seq::Shared<kNT> seq;
  team::Lds tl;
  float red[4][kNT / 64];
  float Slist[kMaxN];
  int par[kMaxN];
  int tk[kMaxN];
  int path[kMaxN];
  float4 stat;  // (max, 1/sum) of the target and the draft row
  int amax;
  unsigned long long kidm[kMaxN];  // children of each node (bit c: node c)
  float2 raw[kMaxN];  // (target, draft) raw values of the current node's rows at each child's token
  float uni[kMaxU];   // the sequence's uniforms (the first kMaxU)
  Args args;          // the launch arguments (stage_args)
  team::Team team;    // this member's team (in LDS, so that no call site keeps it in scratch)
};

__device__ __forceinline__ const float *trow(const Args &a, int b, int n) {
  return a.tgt + (long long)b * a.t_sb + (long long)n * a.t_sn;
}
__device__ __forceinline__ const float *drow(const Args &a, int b, int n) {
  return a.drf + (long long)b * a.d_sb + (long long)n * a.d_sn;
}

// This member's slice [lo, hi) of a row (a multiple of 4 elements long).
__device__ __forceinline__ void slice(const Args &a, const team::Team &tm, long long &lo,
                                      long long &hi) {
  const long long L = ((a.V + tm.G - 1) / tm.G + 3) / 4 * 4;
  lo = min((long long)a.V, (long long)tm.m * L);
  hi = min((long long)a.V, lo + L);
}

// A partial sum exp2((x - m) c) over values of maximum m, rescaled to the
// larger maximum M (0 for an empty partial, m = -inf).
__device__ __forceinline__ float rescale_sum(float m, float s, float M, float c) {
  return (m == -INFINITY) ? 0.0f : s * __builtin_amdgcn_exp2f((m - M) * c);
}

__device__ __forceinline__ float wave_max_f32(float x) {
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) x = fmaxf(x, __shfl_xor(x, k, 64));
  return x;
}
__device__ __forceinline__ float wave_sum_f32(float x) {
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) x += __shfl_xor(x, k, 64);
  return x;
}

// Block-wide (max, sum exp2) of two rows from every thread's partials (m, s):
// the block maximum first (a maximum needs no order), then every thread's sum
// rescaled to it once and summed over lanes (xor butterfly), then over waves
// in order: (m_t, s_t, m_d, s_d).  A merge per butterfly step and per wave
// would cost two exponentials each on one long dependent chain.  Ends with a
// barrier.
__device__ float4 block_ms2(float mt, float st, float md, float sd, float (&red)[4][kNT / 64],
                            float c) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float wmt = wave_max_f32(mt), wmd = wave_max_f32(md);
  if (lane == 0) {
    red[0][wave] = wmt;
    red[2][wave] = wmd;
  }
  __syncthreads();
  float Mt = red[0][0], Md = red[2][0];
#pragma unroll
  for (int w = 1; w < kNT / 64; ++w) {
    Mt = fmaxf(Mt, red[0][w]);
    Md = fmaxf(Md, red[2][w]);
  }
  const float wst = wave_sum_f32(rescale_sum(mt, st, Mt, c));
  const float wsd = wave_sum_f32(rescale_sum(md, sd, Md, c));
  if (lane == 0) {
    red[1][wave] = wst;
    red[3][wave] = wsd;
  }
  __syncthreads();
  float St = 0.0f, Sd = 0.0f;
#pragma unroll
  for (int w = 0; w < kNT / 64; ++w) {
    St += red[1][w];
    Sd += red[3][w];
  }
  __syncthreads();
  return make_float4(Mt, St, Md, Sd);
}

// (max, sum exp2((x - max) c)) of t[lo, hi) and of d[lo, hi) (d may be
// NULL), block-wide, in a fixed order: (m_t, s_t, m_d, s_d).  Both rows'
// loads are issued together.
__device__ __attribute__((noinline)) float4 slice_ms2(const Args &a, const float *t, const float *d, long long lo,
                            long long hi, Smem &sm) {
  const int tid = threadIdx.x;
  const float c = a.c;
  float mt = -INFINITY, st = 0.0f, md = -INFINITY, sd = 0.0f;
  auto update = [c](float &m, float &s, float v0, float v1, float v2, float v3) {
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
    // 16-byte loads; lo and hi are multiples of 4 (a.vec implies V % 4 == 0).
    // Every round issues all U loads of each row before the first use (a
    // lane past the slice end reloads the last vector and skips it), so a
    // slice of up to U * kNT vectors costs one load latency, not one per
    // vector a lane owns.
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 *t4 = reinterpret_cast<const f32x4 *>(t + lo);
    const f32x4 *d4 = d ? reinterpret_cast<const f32x4 *>(d + lo) : t4;
    const int n4 = (int)((hi - lo) / 4);
    constexpr int U = 4;
    for (int i0 = 0; i0 < n4; i0 += U * kNT) {
      f32x4 vt[U], vd[U];
#pragma unroll
      for (int u = 0; u < U; ++u) vt[u] = t4[min(i0 + u * kNT + tid, n4 - 1)];
      if (d) {
#pragma unroll
        for (int u = 0; u < U; ++u) vd[u] = d4[min(i0 + u * kNT + tid, n4 - 1)];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i0 + u * kNT + tid < n4) update(mt, st, vt[u][0], vt[u][1], vt[u][2], vt[u][3]);
      if (d) {
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (i0 + u * kNT + tid < n4) update(md, sd, vd[u][0], vd[u][1], vd[u][2], vd[u][3]);
      }
    }
  } else {
    auto upd1 = [c](float &m, float &s, float v) {
      if (v > m) {
        s *= __builtin_amdgcn_exp2f((m - v) * c);
        m = v;
      }
      const float ms = (m == -INFINITY) ? 0.0f : m;
      s += __builtin_amdgcn_exp2f((v - ms) * c);
    };
    for (long long i = lo + tid; i < hi; i += kNT) {
      upd1(mt, st, t[i]);
      if (d) upd1(md, sd, d[i]);
    }
  }
  return block_ms2(mt, st, md, sd, sm.red, c);
}

// The members' (max, sum) partials p combined (the team maximum, then the
// rescaled sums in member order): sm.stat = (M_t, 1/S_t, M_d, 1/S_d).  Ends
// with a barrier.
template <class SM>
__device__ void team_combine_stats(const Args &a, team::Team &team_ref, SM &sm, float4 p) {
  team::Team tm = team_ref;  // a register copy (see team_seq_r)
  team::exchange(tm, sm.tl, team::f4u(p));
  if (threadIdx.x == 0) {
    // the team maximum, then each member's sum rescaled to it, in member order
    float Mt = -INFINITY, Md = -INFINITY;
    for (int j = 0; j < tm.G; ++j) {
      const float4 v = team::u4f(sm.tl.got[j][0]);
      Mt = fmaxf(Mt, v.x);
      Md = fmaxf(Md, v.z);
    }
    float St = 0.0f, Sd = 0.0f;
    for (int j = 0; j < tm.G; ++j) {
      const float4 v = team::u4f(sm.tl.got[j][0]);
      St += rescale_sum(v.x, v.y, Mt, a.c);
      Sd += rescale_sum(v.z, v.w, Md, a.c);
    }
    sm.stat = make_float4(Mt, 1.0f / St, Md, 1.0f / Sd);
  }
  team_ref.nb = tm.nb;
  __syncthreads();
}

// Softmax statistics of the target row (and the draft row when `d` is set),
// reduced over the team in member order: sm.stat = (M_t, 1/S_t, M_d, 1/S_d).
__device__ void team_stats(const Args &a, team::Team &tm, Smem &sm, const float *t,
                           const float *d) {
  long long lo, hi;
  slice(a, tm, lo, hi);
  const float4 p = slice_ms2(a, t, d, lo, hi, sm);
  team_combine_stats(a, tm, sm, p);
}

__device__ Dist row_dist(const Args &a, const float *row, float M, float invS) {
  Dist d;
  d.p = row;
  d.c = a.c;
  d.logits = a.logits;
  d.M = a.logits ? M : 0.0f;
  d.invS = a.logits ? invS : 1.0f;
  return d;
}

// This member's slice of the probabilities the walk used.
__device__ void write_probs(const Args &a, const team::Team &tm, const Dist &d, float *dst) {
  if (!dst) return;
  long long lo, hi;
  slice(a, tm, lo, hi);
  for (long long i = lo + threadIdx.x; i < hi; i += kNT) dst[i] = d(i);
}

// First index of the largest probability (std::max_element) over the team:
// this member scans [lo, hi), val(i) the probability of index i.
template <class SM, class Val>
__device__ int team_argmax(const Args &a, team::Team &team_ref, SM &sm, long long lo, long long hi,
                           const Val &val) {
  team::Team tm = team_ref;  // a register copy (see team_seq_r)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (long long i = lo + tid; i < hi; i += kNT) {
    const float v = val(i);
    if (v > bv) {  // strided: indices increase, so ">" keeps the first max
      bv = v;
      bi = (int)i;
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
  if (lane == 0) {
    sm.red[0][wave] = bv;
    sm.red[1][wave] = __int_as_float(bi);
  }
  __syncthreads();
  if (tid == 0) {
    float v = sm.red[0][0];
    int ix = __float_as_int(sm.red[1][0]);
    for (int w = 1; w < kNT / 64; ++w) {
      const float v2 = sm.red[0][w];
      const int i2 = __float_as_int(sm.red[1][w]);
      if (v2 > v || (v2 == v && i2 < ix)) {
        v = v2;
        ix = i2;
      }
    }
    sm.red[2][0] = v;
    sm.red[3][0] = __int_as_float(ix);
  }
  __syncthreads();
  team::exchange(tm, sm.tl, make_uint4(__float_as_uint(sm.red[2][0]), __float_as_uint(sm.red[3][0]), 0u, 0u));
  if (tid == 0) {
    float v = __uint_as_float(sm.tl.got[0][0].x);
    int ix = (int)sm.tl.got[0][0].y;
    for (int j = 1; j < tm.G; ++j) {
      const float v2 = __uint_as_float(sm.tl.got[j][0].x);
      const int i2 = (int)sm.tl.got[j][0].y;
      if (v2 > v || (v2 == v && i2 < ix)) {
        v = v2;
        ix = i2;
      }
    }
    sm.amax = (ix == 0x7fffffff) ? 0 : ix;
  }
  team_ref.nb = tm.nb;
  __syncthreads();
  return sm.amax;
}

// ---------------------------------------------------------------------------
// Resident rows.  When a member's share of a row fits in kLCap elements, the
// node's rows are read from HBM once, by the statistics pass, into LDS as
// probabilities (P: target, Q: draft), and every exact pass evaluates its
// elements there: the residual terms max(0, P - Q) or the inverse CDF of P.
// After a residual sum S > 1e-6 is applied, P becomes max(0, P - Q) / S in
// place -- the fp32 operations of Resid::eval (and of the oracle's residual
// update), in the same order -- so an exact pass never divides per element
// and never reads HBM.
// ---------------------------------------------------------------------------
constexpr int kRTile = seq::Shared<kNT>::kTile;  // 16 consecutive elements per thread
constexpr int kLCap = kNT * kRTile;               // elements of a row per member (16384)

struct __align__(16) SmemR {
  float P[kLCap];  // this member's share of the residual r^(k) (target probabilities at k = 0)
  float Q[kLCap];  // ... of the draft probabilities
  seq::Inc tI[kNT];
  int16_t treg[kNT];
  seq::Inc wI[kNT / 64];
  int16_t wreg[kNT / 64];
  uint8_t wserial[kNT / 64];
  float wscan[kNT / 64];
  float s;
  long long found;
  int ctl[4];                  // share-function analysis: first real tile, break, ...
  seq::Inc w0[kNT / 64], w1[kNT / 64];  // per-wave compositions of runs 0 and 1
  uint32_t rec[team::kMaxG][team::kRecWords];  // the members' run-1 records
  team::Lds tl;
  float red[4][kNT / 64];
  float Slist[kMaxN];
  int par[kMaxN];
  int tk[kMaxN];
  int path[kMaxN];
  float4 stat;
  int amax;
  unsigned long long kidm[kMaxN];  // children of each node (bit c: node c)
  float2 raw[kMaxN];
  float uni[kMaxU];
  Args args;
  team::Team team;
};

// Share layout: element e of a share sits in tile e / 16, and the tile's
// four 16-byte chunks are XOR-swizzled by the tile index, so that 16
// consecutive tiles' chunk c (one thread each: a ds_read_b128 of 16 lanes),
// and the 16 elements of one tile (a serial replay), both fall in distinct
// LDS banks.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int chunk_off(int tile, int c) {
  return tile * kRTile + ((c ^ (((tile >> 1) ^ (tile >> 3)) & 3)) << 2);
}
__device__ __forceinline__ int phys(int e) { return chunk_off(e >> 4, (e >> 2) & 3) + (e & 3); }
__device__ __forceinline__ CFA_LDS f32x4 *lds4(float *p) { return (CFA_LDS f32x4 *)p; }
__device__ __forceinline__ const CFA_LDS f32x4 *lds4(const float *p) {
  return (const CFA_LDS f32x4 *)p;
}
__device__ __forceinline__ float lds1(const float *p) { return *(const CFA_LDS float *)p; }

// This member's share [lo, lo + n) of a row in resident mode (shares are a
// multiple of the tile long; the host checks that they fit kLCap).
__device__ __forceinline__ void rslice(const Args &a, const team::Team &tm, long long &lo, int &n) {
  const long long L = ((a.V + tm.G - 1) / tm.G + kRTile - 1) / kRTile * kRTile;
  lo = min((long long)a.V, (long long)tm.m * L);
  n = (int)(min((long long)a.V, lo + L) - lo);
}

// Loads this member's share of row t (and of row d when set) into sm.P
// (sm.Q), zero past its end, as raw values.  With logits, the rows' softmax
// statistics are reduced over the team into sm.stat; convert_share turns the
// share into probabilities when a pass first needs them.  Ends with a
// barrier.
__device__ __attribute__((noinline)) void load_rows_r(const Args &a, team::Team &team_ref, SmemR &sm,
                                                     const float *t, const float *d,
                                                     unsigned long long kids) {
  team::Team tm = team_ref;  // a register copy (see team_seq_r)
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x;
  long long lo;
  int n;
  rslice(a, tm, lo, n);
  const float c = a.c;
  const bool lg = a.logits != 0;
  float mt = -INFINITY, st = 0.0f, md = -INFINITY, sd = 0.0f;
  auto upd = [c](float &m, float &s, float v) {
    if (v > m) {
      s *= __builtin_amdgcn_exp2f((m - v) * c);
      m = v;
    }
    const float ms = (m == -INFINITY) ? 0.0f : m;
    s += __builtin_amdgcn_exp2f((v - ms) * c);
  };
  constexpr int U = kLCap / (4 * kNT);  // 16-byte vectors per thread and row
  // thread c < N: the raw values of the two rows at child c's token (an
  // invalid token reads index 0), issued behind the share's loads
  const bool want = d && tid < a.N && ((kids >> tid) & 1ull);
  float2 raw = make_float2(0.0f, 0.0f);
  if (a.vec) {
    // n % 4 == 0 (V % 4 == 0 and lo % 16 == 0); every load issued before
    // the first use
    typedef const f32x4 __attribute__((address_space(1))) gf32x4;
    const int n4 = n / 4;
    gf32x4 *t4 = (gf32x4 *)(t + lo);
    gf32x4 *d4 = d ? (gf32x4 *)(d + lo) : t4;
    f32x4 vt[U], vd[U];
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = tid + u * kNT;
      vt[u] = i < n4 ? t4[i] : zero;
      vd[u] = (d && i < n4) ? d4[i] : zero;
    }
    if (want) {
      const int x = sm.tk[tid];
      const int xs = (x >= 0 && x < a.V) ? x : 0;
      raw = make_float2(((const float __attribute__((address_space(1))) *)t)[xs],
                        ((const float __attribute__((address_space(1))) *)d)[xs]);
    }
    // the thread's maxima first, then its sums of exponentials against them
    // (no rescaling on the way)
    auto max4 = [](f32x4 v) { return fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])); };
    auto ex4 = [c](f32x4 v, float m) {
      return (__builtin_amdgcn_exp2f((v[0] - m) * c) + __builtin_amdgcn_exp2f((v[1] - m) * c)) +
             (__builtin_amdgcn_exp2f((v[2] - m) * c) + __builtin_amdgcn_exp2f((v[3] - m) * c));
    };
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = tid + u * kNT;  // vector i: chunk i % 4 of tile i / 4
      *lds4(sm.P + chunk_off(i >> 2, i & 3)) = vt[u];
      if (d) *lds4(sm.Q + chunk_off(i >> 2, i & 3)) = vd[u];
      if (i < n4) {
        mt = fmaxf(mt, max4(vt[u]));
        if (d) md = fmaxf(md, max4(vd[u]));
      }
    }
    if (lg) {
      const float bt = (mt == -INFINITY) ? 0.0f : mt, bd = (md == -INFINITY) ? 0.0f : md;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (tid + u * kNT < n4) {  // the two rows' sums interleave
          st += ex4(vt[u], bt);
          if (d) sd += ex4(vd[u], bd);
        }
      }
    }
  } else {
    if (want) {
      const int x = sm.tk[tid];
      const int xs = (x >= 0 && x < a.V) ? x : 0;
      raw = make_float2(t[xs], d[xs]);
    }
    for (int e = tid; e < kLCap; e += kNT) {
      const float x = e < n ? t[lo + e] : 0.0f;
      sm.P[phys(e)] = x;
      if (lg && e < n) upd(mt, st, x);
      if (d) {
        const float y = e < n ? d[lo + e] : 0.0f;
        sm.Q[phys(e)] = y;
        if (lg && e < n) upd(md, sd, y);
      }
    }
  }
  if (want) sm.raw[tid] = raw;
  if (lg) team_combine_stats(a, tm, sm, block_ms2(mt, st, md, sd, sm.red, c));
  team_ref.nb = tm.nb;
  __syncthreads();
}

// The loaded share as probabilities, exp2((x - M) c) * (1 / S) as
// Dist::eval rounds it (logits input; probabilities are loaded as they
// are).  Ends with a barrier.
__device__ __attribute__((noinline)) void convert_share(const Args &a, const team::Team &tm,
                                                       SmemR &sm, bool with_d) {
  if (!a.logits) return;
  long long lo;
  int n;
  rslice(a, tm, lo, n);
  const float4 S = sm.stat;
  const float c = a.c;
  // this thread's tile; elements past n stay zero
  const int tile = threadIdx.x, j0 = tile * kRTile;
  f32x4 pv[kRTile / 4], qv[kRTile / 4];
#pragma unroll
  for (int k = 0; k < kRTile / 4; ++k) {
    pv[k] = *lds4(sm.P + chunk_off(tile, k));
    if (with_d) qv[k] = *lds4(sm.Q + chunk_off(tile, k));
  }
  auto cv = [c, n](float x, float M, float invS, int j) {
    return j < n ? __builtin_amdgcn_exp2f((x - M) * c) * invS : 0.0f;
  };
#pragma unroll
  for (int k = 0; k < kRTile / 4; ++k) {
    f32x4 p, q;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      p[w] = cv(pv[k][w], S.x, S.y, j0 + 4 * k + w);
      if (with_d) q[w] = cv(qv[k][w], S.z, S.w, j0 + 4 * k + w);
    }
    *lds4(sm.P + chunk_off(tile, k)) = p;
    if (with_d) *lds4(sm.Q + chunk_off(tile, k)) = q;
  }
  __syncthreads();
}

// The values of tile `tile` (elements 16 tile .. 16 tile + 15) of this
// member's share for an exact pass: max(0, P - Q) (the residual terms of
// speculative.cpp:33) or P.
__device__ __forceinline__ void share_vals(const SmemR &sm, bool resid, int tile, float (&v)[kRTile]) {
#pragma unroll
  for (int k = 0; k < kRTile / 4; ++k) {
    const f32x4 p = *lds4(sm.P + chunk_off(tile, k));
    if (resid) {
      const f32x4 q = *lds4(sm.Q + chunk_off(tile, k));
#pragma unroll
      for (int w = 0; w < 4; ++w) v[4 * k + w] = relu_ref(p[w] - q[w]);
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) v[4 * k + w] = p[w];
    }
  }
}

// Serial replay of tile `tile` of the share (wave-uniform): lane k < 16
// evaluates element k, the adds take the values lane by lane.
__device__ long long serial_tile_r(const SmemR &sm, bool resid, int tile, float &s, bool cdf,
                                   float r, long long blk0) {
  const int j = phys(tile * kRTile + (seq::lane_id() & (kRTile - 1)));
  const float v = resid ? relu_ref(lds1(sm.P + j) - lds1(sm.Q + j)) : lds1(sm.P + j);
  float x[kRTile];
#pragma unroll
  for (int k = 0; k < kRTile; ++k)
    x[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), k));
  const int k = seq::replay16(x, s, cdf, r);
  return k < 0 ? -1 : blk0 + (long long)tile * kRTile + k;
}

// Walk this member's share exactly from sm.s (wave 0 executes, as
// seq::sweep_block over the functions block_functions_v wrote); updates sm.s
// and sm.found.
__device__ void sweep_share(SmemR &sm, bool resid, long long blk0, bool cdf, float r) {
  using namespace seq;
  float s = sm.s;
  auto tile_desc = [&](int w) {
    return [&sm, w, resid, cdf, r, blk0](int i, float &ss) -> long long {
      return serial_tile_r(sm, resid, w * 64 + i, ss, cdf, r, blk0);
    };
  };
  auto wave_item = [&sm](int i, int &reg) -> Inc {
    reg = sm.wreg[i];
    return sm.wI[i];
  };
  // (a wave crossing several binades is walked tile by tile as well: from
  // LDS a crossing tile's serial replay is cheaper than the wave's)
  auto wave_desc = [&](int w, float &ss) -> long long {
    auto tile_item = [&sm, w](int i, int &reg) -> Inc {
      reg = sm.treg[w * 64 + i];
      return sm.tI[w * 64 + i];
    };
    return walk(64, ss, cdf, r, tile_item, tile_desc(w));
  };
  const long long found = walk(kNT / 64, s, cdf, r, wave_item, wave_desc);
  if (lane_id() == 0) {
    sm.s = s;
    if (found >= 0) sm.found = found;
  }
}

// team::team_seq over the resident shares: the exact left-to-right fp32
// accumulation of max(0, P - Q) (resid; sum mode) or of P (CDF mode: *idx =
// the first index i with r <= s_i, or -1), with the same early exit.  Every
// thread of every member calls it with the same arguments.
template <class Early = team::NoEarlyExit>
__device__ __attribute__((noinline)) float team_seq_r(const Args &a, team::Team &team_ref, SmemR &sm,
                                                      bool resid, bool cdf, float r,
                                                      long long *idx,
                                                      Early early = Early()) {
  using namespace seq;
  // a copy in registers: the caller's object is in its stack, which every
  // store through a generic pointer could alias (each use would reload it)
  team::Team tm = team_ref;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const unsigned tag = ++tm.pass;  // the workspace starts at zero: 0 is never a tag
  long long lo;
  int n;
  rslice(a, tm, lo, n);

  // A: the share's approximate sum (thread tiles, wave scans, waves in order)
  float T = 0.0f;
  {
    float v[kRTile];
    share_vals(sm, resid, tid, v);
    float A = 0.0f;
#pragma unroll
    for (int k = 0; k < kRTile; ++k) A += v[k];
    const float incl = wave_incl_scan_f32(A);
    if (lane == 63) sm.wscan[wave] = incl;
    __syncthreads();
    for (int q = 0; q < kNT / 64; ++q) T += sm.wscan[q];
    __syncthreads();
  }
  team::exchange(tm, sm.tl, make_uint4(f2u(T), 0u, 0u, 0u));
  float E = 0.0f;
  for (int j = 0; j < tm.m; ++j) E += u2f(sm.tl.got[j][0].x);
  if (!cdf) {
    float tot = 0.0f;
    for (int j = 0; j < tm.G; ++j) tot += u2f(sm.tl.got[j][0].x);
    // per member: 16 sequential adds per thread, a 6-level wave scan and 16
    // waves; then the G members
    if (early(tot, (kRTile + 6 + kNT / 64 + 1) + tm.G)) {
      if (idx) *idx = -1;
      team_ref.nb = tm.nb;
      team_ref.pass = tm.pass;
      __syncthreads();
      return -1.0f;
    }
  }

  // B: tile / wave functions from the guess E, and the share as a function
  // of its entry value: kind 1, one run of tiles in region r0; kind 2, run 0
  // in region r0, a break tile (straddling a region boundary, or the first
  // tile of another region) replayed serially from its published values,
  // and run 1 in region r1; kind 0, neither (the owner sweeps the share).
  {
    float v[kRTile];
    share_vals(sm, resid, tid, v);
    team::block_functions_v<kNT>(sm, v, E);
  }
  // Share 0 enters at exactly 0 and crosses a binade every doubling of the
  // running value: its owner publishes kind 0, sweeps it at once (it needs
  // nothing from the others) and hands the exit value on, and collects the
  // other members' functions afterwards.
  float s = 0.0f;
  long long found = -1;
  int j0 = 0;
  if (tm.m == 0) {
    team::exchange_publish(tm, make_uint4(0u, 0u, (uint32_t)kAnyRegion, 0u));
    if (tid == 0) {
      sm.s = 0.0f;
      sm.found = -1;
    }
    __syncthreads();
    if (wave == 0) sweep_share(sm, resid, lo, cdf, r);
    __syncthreads();
    s = sm.s;
    found = sm.found;
    team::put_hand(tm, 1, tag, s, found);
    team::exchange_collect(tm, sm.tl);
    j0 = 1;
  } else {
    // the first tile of the share (in tile order) meeting a condition: one
    // LDS atomic per wave, from its first lane that meets it
    auto first_of = [&](bool c, int slot) {
      const unsigned long long m = __ballot(c);
      if (m && lane == (int)__builtin_ctzll(m)) atomicMin(&sm.ctl[slot], tid);
    };
    const Inc f = sm.tI[tid];
    const int reg = sm.treg[tid];
    const bool bad = f.e == kBad;
    if (tid < 4) sm.ctl[tid] = tid < 3 ? kNT : 0;
    __syncthreads();
    first_of(bad || reg != kAnyRegion, 0);  // the first real tile
    __syncthreads();
    const int fr = sm.ctl[0];
    const int r0 = fr < kNT ? sm.treg[fr] : kAnyRegion;
    first_of(bad || (reg != kAnyRegion && reg != r0), 1);  // the break
    __syncthreads();
    const int brk = sm.ctl[1];
    first_of(tid > brk && (bad || reg != kAnyRegion), 2);  // the first real tile after it
    __syncthreads();
    const int fa = sm.ctl[2];
    const int r1 = fa < kNT ? sm.treg[fa] : kAnyRegion;
    if (__ballot(tid > brk && (bad || (reg != kAnyRegion && reg != r1))) && lane == 0)
      sm.ctl[3] = 1;  // not two runs
    const Inc w0 = wave_incl_compose(tid < brk ? f : inc_identity());
    const Inc w1 = wave_incl_compose((tid > brk && !bad) ? f : inc_identity());
    if (lane == 63) {
      sm.w0[wave] = w0;
      sm.w1[wave] = w1;
    }
    __syncthreads();
    const int kind = brk >= kNT ? 1 : (sm.ctl[3] ? 0 : 2);
    Inc F0 = inc_identity(), F1 = inc_identity();
    if (tid == 0) {
      for (int w = 0; w < kNT / 64; ++w) {
        F0 = compose(F0, sm.w0[w]);
        F1 = compose(F1, sm.w1[w]);
      }
      sm.tl.got[0][1] = make_uint4(F0.e, F0.o, (uint32_t)r0, (uint32_t)kind);  // scratch
      sm.w0[0] = F1;
    }
    __syncthreads();
    if (kind == 2 && tid < team::kRecWords) {
      // the record: run 1's function and region, the break tile, its values
      uint32_t w;
      if (tid == 0) w = sm.w0[0].e;
      else if (tid == 1) w = sm.w0[0].o;
      else if (tid == 2) w = (uint32_t)r1;
      else if (tid == 3) w = (uint32_t)brk;
      else {
        const int j = phys(brk * kRTile + (tid - 4));
        w = f2u(resid ? relu_ref(lds1(sm.P + j) - lds1(sm.Q + j)) : lds1(sm.P + j));
      }
      team::st64(&tm.st->rec[tm.m][tid], ((unsigned long long)tag << 32) | w);
    }
    team::exchange(tm, sm.tl, sm.tl.got[0][1]);
  }
  // the records of the shares that published two runs (bounded waits on
  // their tags)
  if (tid < team::kMaxG * team::kRecWords) {
    const int j = tid / team::kRecWords, w = tid % team::kRecWords;
    if (j < tm.G && sm.tl.got[j][0].w == 2u) {
      unsigned long long x = 0;
      long spins = 0;
      for (;;) {
        x = team::ld64(&tm.st->rec[j][w]);
        if ((unsigned)(x >> 32) == tag) break;
        if (sm.tl.failed || ++spins > team::kSpinLimit || team::error_set(tm.err)) {
          sm.tl.failed = 1;
          team::set_error(tm.err);
          x = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      sm.rec[j][w] = (uint32_t)x;
    }
  }
  __syncthreads();
  const long long L = ((a.V + tm.G - 1) / tm.G + kRTile - 1) / kRTile * kRTile;

  // C: walk the shares from the exact running value
  // one run of region reg from the exact value v (false: it does not apply)
  auto run = [](Inc F, int reg, float &v) -> bool {
    if (reg == kAnyRegion) return true;
    const int rs = region_of(v);
    if (rs != reg) return false;
    const uint32_t au = units_of(v, rs);
    const uint32_t inc = inc_at(F, au);
    if (au + inc > kUnitsTop) return false;
    v = value_of(au + inc, rs);
    return true;
  };
  for (int j = j0; j < tm.G && !(cdf && found >= 0); ++j) {
    const uint4 fj = sm.tl.got[j][0];
    bool applies = false;
    float snext = s;
    if (fj.w == 1u) {
      applies = run(Inc{fj.x, fj.y}, (int)fj.z, snext) && !(cdf && r <= snext);
    } else if (fj.w == 2u && run(Inc{fj.x, fj.y}, (int)fj.z, snext) && !(cdf && r <= snext)) {
      // run 0 applied; the break tile serially, then run 1
      const int brk = (int)sm.rec[j][3];
      float x[kRTile];
#pragma unroll
      for (int k = 0; k < kRTile; ++k) x[k] = u2f(sm.rec[j][4 + k]);
      const int k = seq::replay16(x, snext, cdf, r);
      if (k >= 0) {  // the draw lands in the break tile
        s = snext;
        found = (long long)j * L + (long long)brk * kRTile + k;
        break;
      }
      applies = run(Inc{sm.rec[j][0], sm.rec[j][1]}, (int)sm.rec[j][2], snext) &&
                !(cdf && r <= snext);
    }
    if (applies) {
      s = snext;
      continue;
    }
    if (j == tm.m) {  // sweep this share exactly from s
      if (tid == 0) {
        sm.s = s;
        sm.found = -1;
      }
      __syncthreads();
      if (wave == 0) sweep_share(sm, resid, lo, cdf, r);
      __syncthreads();
      s = sm.s;
      found = sm.found;
      team::put_hand(tm, j + 1, tag, s, found);
      __syncthreads();
    } else {
      team::get_hand(tm, sm.tl, j + 1, tag, s, found);
    }
    if (cdf && found >= 0) break;
  }
  (void)n;
  if (idx) *idx = found;
  __syncthreads();  // every thread has read sm.found above
  if (tid == 0) sm.found = found;  // the CDF hit, for callers that read it from LDS
  team_ref.nb = tm.nb;
  team_ref.pass = tm.pass;
  __syncthreads();
  return s;
}

// r^(k+1) = max(0, r^(k) - q) / S in place over this member's share (the
// order of operations of Resid::eval).  Ends with a barrier.
__device__ __attribute__((noinline)) void normalize_share(SmemR &sm, float S) {
  // element-wise at every position (P and Q share the layout)
  f32x4 pv[kRTile / 4], qv[kRTile / 4];
#pragma unroll
  for (int k = 0; k < kRTile / 4; ++k) {
    pv[k] = *lds4(sm.P + 4 * (threadIdx.x + k * kNT));
    qv[k] = *lds4(sm.Q + 4 * (threadIdx.x + k * kNT));
  }
#pragma unroll
  for (int k = 0; k < kRTile / 4; ++k) {
    f32x4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r[w] = relu_ref(pv[k][w] - qv[k][w]) / S;
    *lds4(sm.P + 4 * (threadIdx.x + k * kNT)) = r;
  }
  __syncthreads();
}

// This member's share of P or Q (the probabilities of a visited row) to dst.
__device__ __attribute__((noinline)) void write_share(const Args &a, const team::Team &tm,
                                                     const float *src, float *dst) {
  if (!dst) return;
  long long lo;
  int n;
  rslice(a, tm, lo, n);
  for (int e = threadIdx.x; e < n; e += kNT) dst[lo + e] = lds1(src + phys(e));
}

// One sequence's walk; every member of the team runs it with the same data.
// RES: the node's rows are resident in LDS (SmemR), else re-read from HBM
// by every exact pass (Smem).
template <bool RES, class SM>
__device__ void walk_sequence(const Args &a, team::Team &tm, SM &sm, int b) {
  const int tid = threadIdx.x;
  const int N = a.N, V = a.V;
  if (tid < N) {
    sm.par[tid] = a.parent[(long long)b * a.parent_sb + tid];
    sm.tk[tid] = a.tok[(long long)b * N + tid];
  }
  if (tid == 0) sm.path[0] = 0;
  const float *Ug = a.U ? a.U + (long long)b * a.n_u : nullptr;
  if (Ug)
    for (int i = tid; i < min(a.n_u, kMaxU); i += kNT) sm.uni[i] = Ug[i];
  __syncthreads();
  // children of every node (bit c of kidm[n]: parent[c] = n with n < c)
  if (tid < N) sm.kidm[tid] = 0ull;
  __syncthreads();
  if (tid > 0 && tid < N) {
    const int pc = sm.par[tid];
    if (pc >= 0 && pc < tid) atomicOr(&sm.kidm[pc], 1ull << tid);
  }
  __syncthreads();
  // draw i: from LDS when staged
  auto U_at = [&](int i) -> float { return i < kMaxU ? sm.uni[i] : Ug[i]; };
  int node = 0, len = 1, draws = 0, fin = -1, eos_acc = 0, status = 0;
  for (;;) {
    // children of `node`, in increasing index order
    const unsigned long long kids = sm.kidm[node];
    __syncthreads();  // every wave is done with the previous node's sm.raw and sm.stat
    const bool leaf = kids == 0;
    const float *tr = trow(a, b, node);
    const float *dr = (leaf || a.greedy) ? nullptr : drow(a, b, node);
    // the rows' raw values at the children's tokens, loaded ahead of the
    // statistics pass (thread c: child c; an invalid token reads index 0);
    // load_rows_r gathers them behind its own loads
    if (!RES && dr && tid < N && ((kids >> tid) & 1ull)) {
      const int x = sm.tk[tid];
      const int xs = (x >= 0 && x < V) ? x : 0;
      sm.raw[tid] = make_float2(tr[xs], dr[xs]);
    }
    // resident rows: whether the share holds probabilities yet (the first
    // pass that reads them converts it; a node whose first child is
    // accepted never does)
    bool conv = false;
    auto ensure_probs = [&]() {
      if constexpr (RES) {
        if (!conv) convert_share(a, tm, sm, dr != nullptr);
        conv = true;
      }
    };
    if constexpr (RES) {
      load_rows_r(a, tm, sm, tr, dr, kids);
    } else {
      if (a.logits) team_stats(a, tm, sm, tr, dr);
      else __syncthreads();
    }
    const float4 st = sm.stat;
    const Dist t = row_dist(a, tr, st.x, st.y);
    float *const pt_out = a.probs_t ? a.probs_t + ((long long)b * N + node) * V : nullptr;
    if constexpr (RES) {
      if (pt_out || a.probs_d) {
        ensure_probs();
        write_share(a, tm, sm.P, pt_out);
      }
    } else if (pt_out) {
      write_probs(a, tm, t, pt_out);
    }
    // the first index of the largest target probability, over the team
    auto argmax_t = [&]() -> int {
      long long lo, hi;
      if constexpr (RES) {
        ensure_probs();
        int n;
        rslice(a, tm, lo, n);
        return team_argmax(a, tm, sm, lo, lo + n,
                           [&sm, lo](long long i) { return lds1(sm.P + phys((int)(i - lo))); });
      } else {
        slice(a, tm, lo, hi);
        return team_argmax(a, tm, sm, lo, hi, t);
      }
    };
    if (leaf) {  // the bonus token
      if (a.greedy) {
        fin = argmax_t();
      } else {
        if (draws >= a.n_u) {
          status = 1;
          break;
        }
        long long idx = -1;
        if constexpr (RES) {
          ensure_probs();
          team_seq_r(a, tm, sm, false, true, U_at(draws++), nullptr);
          idx = sm.found;  // the hit, as team_seq_r left it in LDS
        } else {
          team::team_seq<kNT>(tm, sm.tl, Resid{t, t, sm.Slist, 0}, V, true, U_at(draws++),
                              sm.seq, &idx);
        }
        fin = (idx < 0) ? V - 1 : (int)idx;
      }
      break;
    }
    int accepted = -1;
    if (a.greedy) {
      const int am = argmax_t();
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
      const Dist d = row_dist(a, dr, st.z, st.w);
      float *const pd_out = a.probs_d ? a.probs_d + ((long long)b * N + node) * V : nullptr;
      if constexpr (RES) write_share(a, tm, sm.Q, pd_out);
      else if (pd_out) write_probs(a, tm, d, pd_out);
      int k = 0;  // applied normalisations of the residual
      for (unsigned long long m = kids; m; m &= m - 1) {
        const int c = __builtin_ctzll(m);
        const int x = sm.tk[c];
        const bool valid = x >= 0 && x < V;
        const int xs = valid ? x : 0;
        (void)xs;
        const Resid r{t, d, sm.Slist, k};
        const float2 raw = sm.raw[c];
        const float p = r.eval(raw);  // r^(k)(x)
        const float q = d.eval(raw.y);
        const float ratio = valid ? ratio_cpp(p, q) : -1.0f;  // an out-of-range id never passes
        if (draws >= a.n_u) {
          status = 1;
          break;
        }
        const float u = U_at(draws++);
        if (u <= ratio) {
          accepted = c;
          break;
        }
        // the next sibling, when its test can be settled from bounds on S
        const unsigned long long rest = m & (m - 1);
        float S;
        if (rest && draws < a.n_u && sm.tk[__builtin_ctzll(rest)] >= 0 &&
            sm.tk[__builtin_ctzll(rest)] < V) {
          const SiblingAccepts early{r, sm.raw[__builtin_ctzll(rest)], U_at(draws), (long long)V};
          if constexpr (RES) {
            ensure_probs();
            S = team_seq_r(a, tm, sm, true, false, 0.0f, nullptr, early);
          } else
            S = team::team_seq<kNT>(tm, sm.tl, ResidX{r}, V, false, 0.0f, sm.seq, nullptr, early);
          if (S < 0.0f) {  // the sibling is accepted for every S in the bounds
            accepted = __builtin_ctzll(rest);
            ++draws;
            break;
          }
        } else {
          if constexpr (RES) {
            ensure_probs();
            S = team_seq_r(a, tm, sm, true, false, 0.0f, nullptr);
          } else
            S = team::team_seq<kNT>(tm, sm.tl, ResidX{r}, V, false, 0.0f, sm.seq, nullptr);
        }
        if (S > 1e-6f) {  // else the residual stays (speculative.cpp:37-40)
          if (tid == 0) sm.Slist[k] = S;
          __syncthreads();
          ++k;
          if constexpr (RES) normalize_share(sm, S);
        }
      }
      if (status) break;
      if (accepted < 0) {
        if (draws >= a.n_u) {
          status = 1;
          break;
        }
        long long idx = -1;
        if constexpr (RES) {
          ensure_probs();
          team_seq_r(a, tm, sm, false, true, U_at(draws++), nullptr);
          idx = sm.found;  // the hit, as team_seq_r left it in LDS
        } else {
          team::team_seq<kNT>(tm, sm.tl, Resid{t, d, sm.Slist, k}, V, true, U_at(draws++),
                              sm.seq, &idx);
        }
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
  if (sm.tl.failed || team::error_set(a.err)) status = 2;  // a team wait timed out
  if (tm.m != 0) return;
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

// The launch arguments, copied once from the kernarg segment into the
// work-group's LDS.  The walk passes them by reference to out-of-line
// functions; a reference to the by-value kernel parameter would make every
// lane keep its own copy in scratch memory.
template <class SM>
__device__ __forceinline__ const Args &stage_args(SM &sm) {
  static_assert(sizeof(Args) % 4 == 0 && sizeof(Args) / 4 <= kNT, "Args copy");
  typedef const uint32_t __attribute__((address_space(4))) kword;
  kword *src = (kword *)__builtin_amdgcn_kernarg_segment_ptr();
  if (threadIdx.x < sizeof(Args) / 4)
    reinterpret_cast<uint32_t *>(&sm.args)[threadIdx.x] = src[threadIdx.x];
  __syncthreads();
  return sm.args;
}

template <bool RES, class SM>
__device__ __forceinline__ void tree_verify_body(SM &sm) {
  const Args &a = stage_args(sm);
  const int team_id = (int)blockIdx.x / a.G;
  if (threadIdx.x == 0) {
    sm.tl.failed = 0;
    sm.team = team::Team{a.teams + team_id, a.err, (int)blockIdx.x % a.G, a.G, 0u, 0u};
  }
  __syncthreads();
  if (team_id >= a.T) return;
  // Functions that exchange work on a register copy and store the
  // exchange and pass counts back before their last barrier.
  team::Team &tm = sm.team;
  for (int b = team_id; b < a.B; b += a.T) {
    walk_sequence<RES>(a, tm, sm, b);
    __syncthreads();
  }
}

// Every exact pass re-reads its elements from HBM (any V).
__global__ __launch_bounds__(kNT) void tree_verify_kernel(Args) {
  __shared__ Smem sm;
  tree_verify_body<false>(sm);
}

// The visited rows stay resident in LDS (a member's share of a row at most
// kLCap elements).
__global__ __launch_bounds__(kNT) void tree_verify_res_kernel(Args) {
  __shared__ SmemR sm;
  tree_verify_body<true>(sm);
}

// Zero the teams' state before the launch.
__global__ __launch_bounds__(256) void clear_kernel(uint4 *p, long long n) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Teams and members for B sequences on `cus` CUs holding `per_cu` work-groups.
struct Plan {
  int G, T;
};
inline Plan plan(int B, int cus, int per_cu) {
  const int slots = max(1, cus * max(1, per_cu));
  int G = team::kMaxG;
  while (G > 1 && (long long)B * G > slots) G >>= 1;
  const int T = max(1, min(B, slots / G));
  return Plan{G, T};
}

}  // namespace treev
}  // namespace cfa

using namespace cfa;

namespace {
// Work-groups of a tree kernel (0: rows re-read, 1: rows resident) one CU
// holds, per device (queried once; threads that race on the first query
// store the same value).
int kernel_per_cu(int which) {
  static std::atomic<int> cache[2][64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  int n = cache[which][dev].load(std::memory_order_relaxed);
  if (n == 0) {
    const void *k = which ? (const void *)treev::tree_verify_res_kernel
                          : (const void *)treev::tree_verify_kernel;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, treev::kNT, 0) != hipSuccess || n < 1)
      n = 1;
    cache[which][dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// CFA_TREE_RESIDENT=0 keeps every vocabulary on the kernel that re-reads
// rows from HBM (the path for shares larger than the LDS holds).
bool resident_allowed() {
  static const bool on = [] {
    const char *v = std::getenv("CFA_TREE_RESIDENT");
    return !(v != nullptr && v[0] == '0');
  }();
  return on;
}
constexpr size_t kErrBytes = 256;

bool cooperative_launch() {
  static const bool on = [] {
    const char *v = std::getenv("CFA_COOPERATIVE_LAUNCH");
    return v != nullptr && v[0] == '1';
  }();
  return on;
}
}  // namespace

extern "C" size_t cfa_tree_verify_workspace_size(int B) {
  if (B <= 0) return 0;
  return kErrBytes + (size_t)B * sizeof(team::State);
}

extern "C" int cfa_tree_verify(const float *target, int64_t t_stride_b, int64_t t_stride_n,
                               const float *draft, int64_t d_stride_b, int64_t d_stride_n,
                               int input_kind, const int32_t *parents, int64_t parents_stride_b,
                               const int32_t *node_tokens, const float *uniforms, int n_uniforms,
                               int B, int N, int V, float temperature, int mode,
                               int32_t eos_token_id, int32_t *out_path, int32_t *out_path_len,
                               int32_t *out_tokens, int32_t *out_num_emitted, int32_t *out_final,
                               int32_t *out_eos, int32_t *out_status, float *out_target_probs,
                               float *out_draft_probs, void *workspace, size_t workspace_bytes,
                               void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (B <= 0 || N <= 0 || N > treev::kMaxN || V <= 0)
    return fail_arg("need B > 0, 0 < N <= 64 and V > 0");
  if (V >= (1 << 24) - 1) return fail_arg("V must be below 16777215");
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
  const int cus = device_cu_count();
  // rows resident in LDS when a member's share of a row fits there
  treev::Plan pl = treev::plan(B, cus, kernel_per_cu(1));
  const long long share = ((long long)(V + pl.G - 1) / pl.G + treev::kRTile - 1) /
                          treev::kRTile * treev::kRTile;
  const bool resident = resident_allowed() && share <= treev::kLCap;
  if (!resident) pl = treev::plan(B, cus, kernel_per_cu(0));
  const size_t need = kErrBytes + (size_t)pl.T * sizeof(team::State);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255))
    return fail_arg("workspace missing, too small or not 256-byte aligned "
                    "(see cfa_tree_verify_workspace_size)");
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
  a.T = pl.T;
  a.G = pl.G;
  a.err = (int *)workspace;
  a.teams = (team::State *)((char *)workspace + kErrBytes);
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
  hipStream_t st = (hipStream_t)stream;
  const long long words = (long long)(need / sizeof(uint4));
  CFA_LAUNCH("tree_verify_clear", treev::clear_kernel,
             dim3((unsigned)std::min<long long>((words + 255) / 256, 1024)), dim3(256), 0, st,
             (uint4 *)workspace, words);
  // A team's members must be resident together.  plan() never asks for more
  // work-groups than the device holds at once for this kernel (occupancy
  // query), so on a device running no other kernel every member is resident
  // from the start; kernels of other streams can only delay a member, and one
  // delayed past the bounded wait makes its team report status 2.
  // hipLaunchCooperativeKernel guarantees residency, but measured on MI355X
  // (ROCm 7) it leaves the process's later dispatches slower for a while
  // (~15 us added to each; the 8B-shape target forward that follows it:
  // 15.3 -> 24.5 ms), and the kernel itself runs slower (B = 8: 0.34 against
  // 0.21 ms), so it is taken only when CFA_COOPERATIVE_LAUNCH=1.
  const dim3 grid((unsigned)(pl.T * pl.G));
  if (cooperative_launch()) {
    void *tok = prof::enabled() ? prof::begin("tree_verify", st) : nullptr;
    void *args[] = {&a};
    const void *k = resident ? (const void *)treev::tree_verify_res_kernel
                             : (const void *)treev::tree_verify_kernel;
    const hipError_t e = hipLaunchCooperativeKernel(k, grid, dim3(treev::kNT), args, 0, st);
    if (tok) prof::end(tok, st);
    if (e != hipSuccess) return fail_hip(e, "tree_verify (cooperative launch)");
  } else if (resident) {
    CFA_LAUNCH("tree_verify", treev::tree_verify_res_kernel, grid, dim3(treev::kNT), 0, st, a);
  } else {
    CFA_LAUNCH("tree_verify", treev::tree_verify_kernel, grid, dim3(treev::kNT), 0, st, a);
  }
  return CFA_OK;
}
