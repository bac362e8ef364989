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
#include <mutex>

#include "abi_internal.hpp"
#include "dist.hpp"
#include "lds_dma.hpp"
#include "seqsum.hpp"

// Every fp32 expression below must round exactly as written (the oracle and
// the reference evaluate t_i - d_i, p / q and x / S as separate roundings).
#pragma clang fp contract(off)

namespace cfa {
namespace chain {

enum Kind : int { kNone = 0, kResid = 1, kPlain = 2, kPyBonus = 3 };

// Exact multi-work-group sampler state (per sequence b).
constexpr int kMwNT = 256;                  // threads per sums / records work-group
constexpr int kMwTile = 16;                 // elements per lane (one tile)
constexpr int kMwChunkTiles = 64;           // tiles per chunk (one wave)
constexpr int kMwChunk = kMwChunkTiles * kMwTile;  // 1024 elements per chunk
constexpr int kMwMaxBad = 64;               // cached serial tiles per row and pass
constexpr int kMwPf = 8;                    // chunks whose tile records the walk prefetches
constexpr int kMwSerialTiles = 4;           // leading tiles of chunk 0 the walk replays serially
// Relative slack within which a tile counts as near a binade boundary (its
// values are cached for the walk).  The approximate prefix that places tiles
// differs from the exact running value by about 2^-15 relatively at V = 128K.
constexpr float kMwNear = 1.0f / 4096.0f;
constexpr int kMwMaxNC = 4096;              // chunks per row (V <= 4M)
struct MwJob {  // what sequence b still has to draw
  int kind, row, n, eos_acc;
  float u;          // the draw's threshold (python mode: see py_threshold)
  float tM, tInvS;  // (max, 1/S) of the target row (logits input)
  float dM, dInvS;  // and of the draft row of a residual draw
  int extra;        // python mode: a bonus draw follows the resample
  float u2;         // and its threshold
  int pad;
};
struct MwRes {  // per sequence: residual sum, fallback flag, drawn index(es)
  float S;
  int fallback, idx, idx2;
};
struct MwRec {  // a tile's function of the entry parity, its region guess, pad = 1: replay
  uint32_t e, o;
  int reg, pad;
};
// A chunk as run 0 (tiles [0, brk)), break tile brk (replayed serially when
// brk_serial, otherwise run 1 starts there in another region) and run 1
// (the rest); brk = -1: one run.  Runs are functions of the entry parity.
// near = 1: the walk will probably go down to this chunk's tiles (it holds a
// tile cached for a serial replay), so the walk prefetches its tile records.
struct MwChunk {
  uint32_t e0, o0, e1, o1;
  int reg0, reg1;
  int brk, brk_serial;
  int status, near, pad[2];
};
struct MwBad {  // a tile the walk will probably replay serially, with its values
  int tile, pad[3];
  float x[kMwTile];
};

struct Args {
  const float *tgt;
  long long t_sb, t_sk;
  const float *drf;
  long long d_sb, d_sk;
  const int32_t *tokens;  // [B,K]
  const float *U;         // [B,ustride]
  int ustride;            // uniforms per sequence: K+1, or K+2 in python mode
  int B, K, V, rpb;       // rows per sequence: K+1 (greedy) or 2K+1
  int draws;              // jobs per input row (sequence b reads row b / draws)
  int R;                  // distinct rows: (B / draws) * rpb
  float c;                // log2(e) / temperature
  int logits;             // 1: inputs are logits
  int mode;               // CFA_MODE_*
  int eos;
  float top_p;
  int top_k;              // > 0: keep only probabilities >= the top_k-th largest
  // partition of the stats / argmax passes: every row in S fixed slices
  long long Vw;  // row length in vector units
  int S;         // slices per row (a function of the shape only)
  int P;         // cpp rules, logits: positions whose rows the first stats pass reads
  float2 *part;  // [R, S] (max logit, sum exp) per (row, slice)
  float2 *apart; // [R, S] (max prob, index as bits) per (row, slice)
  int4 *dec;     // [B] {n_b, kind, row, eos_accepted}
  float *ufin;   // [B]
  // exact multi-work-group sampler (see "mw" below)
  int vec;                // rows are 16-byte aligned with V % 4 == 0
  int NC;                 // chunks per row
  MwJob *jobs;            // [B]
  MwRes *res;             // [B]
  float *csum_x, *csum_t; // [B, NC] approximate chunk sums
  MwChunk *crec;          // [2, B, NC]   chunk structure, per pass
  MwRec *trec;            // [2, B, NC*64] tile functions, per pass
  int *badcnt;            // [2, B]
  MwBad *bad;             // [2, B, kMwMaxBad]
  float *x0;              // [2, B, kMwChunk] chunk 0's element values per pass
  unsigned long long *flags;  // [B, NC] look-back words of the first exact pass
  unsigned long long *tsync;  // [B, 2] mw_tail_kernel: S published, CDF shares done
  float *s0;              // [B] sum pass: the exact running value after chunk 0
  int mw_reset;           // the first statistics pass zeroes flags and badcnt
  float *rawtok;          // [R] head pass: a row's raw logit at its position's draft token
  int32_t *out_accept_len, *out_tokens, *out_num_emitted, *out_final, *out_eos;
};

// Row j of input row group ub (a sequence's K+1 target rows, then its K draft rows).
__device__ __forceinline__ const float *row_ptr_u(const Args &a, int ub, int j) {
  return j <= a.K ? a.tgt + (long long)ub * a.t_sb + (long long)j * a.t_sk
                  : a.drf + (long long)ub * a.d_sb + (long long)(j - a.K - 1) * a.d_sk;
}
// Row j of job b.
__device__ __forceinline__ const float *row_ptr(const Args &a, int b, int j) {
  return row_ptr_u(a, b / a.draws, j);
}

// (max, 1/S) of row r from its slices' partials, combined in slice order
// (the same for whichever pass computed the row).  Up to kFastS slices
// (every row at C2 has 2) the partials load in one round before any use;
// the arithmetic is the same, in the same order, either way.
constexpr int kFastS = 4;
struct RowParts {
  float2 p[kFastS];
};
__device__ __forceinline__ void row_parts_load(const Args &a, int r, RowParts &q) {
#pragma unroll
  for (int w = 0; w < kFastS; ++w)
    if (w < a.S) q.p[w] = a.part[(long long)r * a.S + w];
}
__device__ __forceinline__ float2 row_parts_stat(const Args &a, const RowParts &q) {
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kFastS; ++w)
    if (w < a.S) M = fmaxf(M, q.p[w].x);
  float S = 0.0f;
#pragma unroll
  for (int w = 0; w < kFastS; ++w)
    if (w < a.S) S += (q.p[w].x == M) ? q.p[w].y : q.p[w].y * __builtin_amdgcn_exp2f((q.p[w].x - M) * a.c);
  return make_float2(M, 1.0f / S);
}
__device__ float2 row_stat(const Args &a, int r) {
  if (a.S <= kFastS) {
    RowParts q;
    row_parts_load(a, r, q);
    return row_parts_stat(a, q);
  }
  const float2 *p = a.part + (long long)r * a.S;
  float M = -INFINITY;
  for (int w = 0; w < a.S; ++w) M = fmaxf(M, p[w].x);
  float S = 0.0f;
  for (int w = 0; w < a.S; ++w) {
    const float2 ms = p[w];
    S += (ms.x == M) ? ms.y : ms.y * __builtin_amdgcn_exp2f((ms.x - M) * a.c);
  }
  return make_float2(M, 1.0f / S);
}

__device__ Dist make_dist_u(const Args &a, int ub, int j) {
  Dist d;
  d.p = row_ptr_u(a, ub, j);
  d.c = a.c;
  d.logits = a.logits;
  d.M = 0.0f;
  d.invS = 1.0f;
  if (a.logits) {
    const float2 st = row_stat(a, ub * a.rpb + j);
    d.M = st.x;
    d.invS = st.y;
  }
  return d;
}
__device__ Dist make_dist(const Args &a, int b, int j) { return make_dist_u(a, b / a.draws, j); }

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

// Streaming 16-byte load: every logit is read once here, so the lines are
// marked non-temporal instead of displacing cached data (on MI355X this
// raises the pass from ~65% to ~75% of HBM peak).
__device__ __forceinline__ float4 ld_stream4(const float4 *p) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4 q = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
  return make_float4(q[0], q[1], q[2], q[3]);
}

// Row sets of a stats pass.  Under the cpp rules with logits input only the
// rows of positions up to a sequence's first rejection are ever read, so
// the first pass takes positions 0 .. P-1 of every sequence ("head"), and
// the second the remaining rows (positions P .. K-1 and the target's row K,
// "tail") of the sequences that accepted all P head positions.
enum RowSet : int { kRowsAll = 0, kRowsHead = 1, kRowsTail = 2 };

// Row id (ub * rpb + j) of entry y of a row set; -1 past its end.
__device__ __forceinline__ int set_row(const Args &a, int set, int y) {
  const int groups = a.R / a.rpb;
  if (set == kRowsAll) return y < a.R ? y : -1;
  const int P = a.P, K = a.K;
  if (set == kRowsHead) {
    const int ub = y / (2 * P), q = y % (2 * P);
    return ub < groups ? ub * a.rpb + (q < P ? q : K + 1 + (q - P)) : -1;
  }
  const int per = 2 * (K - P) + 1, ub = y / per, q = y % per;
  return ub < groups ? ub * a.rpb + (q <= K - P ? P + q : K + 1 + P + (q - (K - P + 1))) : -1;
}

// Whether row group ub accepted head position i under the cpp rules
// (speculative.cpp:66-80: position i takes the i-th uniform when all before
// it were accepted, and an accepted EOS ends the walk), from the head pass's
// statistics and the raw logit at the draft token it recorded.
__device__ __forceinline__ bool head_accepts(const Args &a, int ub, int i) {
  const int rt = ub * a.rpb + i, rd = ub * a.rpb + a.K + 1 + i;
  const int traw = a.tokens[(long long)ub * a.K + i];
  const float u = a.U[(long long)ub * a.ustride + i];
  const float2 st = row_stat(a, rt), sd = row_stat(a, rd);
  const float pt = __builtin_amdgcn_exp2f((a.rawtok[rt] - st.x) * a.c) * st.y;
  const float qd = __builtin_amdgcn_exp2f((a.rawtok[rd] - sd.x) * a.c) * sd.y;
  const bool valid = traw >= 0 && traw < a.V;
  return valid && u <= ratio_cpp(pt, qd) && traw != a.eos;
}

// Whether row group ub accepted every head position (head_accepts for each,
// the same operations in the same order): with P <= kFastP and S <= kFastS
// every load of the test is issued before the first use, one round of
// loads instead of a round trip per position and slice.
constexpr int kFastP = 3;
__device__ bool head_all_accept(const Args &a, int ub) {
  if (a.P > kFastP || a.S > kFastS) {
    bool ok = true;
    for (int i = 0; i < a.P; ++i) ok &= head_accepts(a, ub, i);
    return ok;
  }
  RowParts qt[kFastP], qd[kFastP];
  float rt[kFastP], rd[kFastP], u[kFastP];
  int tk[kFastP];
#pragma unroll
  for (int i = 0; i < kFastP; ++i) {
    if (i < a.P) {
      const int r_t = ub * a.rpb + i, r_d = ub * a.rpb + a.K + 1 + i;
      row_parts_load(a, r_t, qt[i]);
      row_parts_load(a, r_d, qd[i]);
      rt[i] = a.rawtok[r_t];
      rd[i] = a.rawtok[r_d];
      tk[i] = a.tokens[(long long)ub * a.K + i];
      u[i] = a.U[(long long)ub * a.ustride + i];
    }
  }
  bool ok = true;
#pragma unroll
  for (int i = 0; i < kFastP; ++i) {
    if (i < a.P) {
      const float2 st = row_parts_stat(a, qt[i]), sd = row_parts_stat(a, qd[i]);
      const float pt = __builtin_amdgcn_exp2f((rt[i] - st.x) * a.c) * st.y;
      const float q = __builtin_amdgcn_exp2f((rd[i] - sd.x) * a.c) * sd.y;
      const bool valid = tk[i] >= 0 && tk[i] < a.V;
      ok &= valid && u[i] <= ratio_cpp(pt, q) && tk[i] != a.eos;
    }
  }
  return ok;
}

// Whether row group ub accepted every head position, i.e. needs its tail
// rows.  Every thread of the work-group gets the answer; every load is
// independent of the others.
template <int NT>
__device__ bool tail_needed(const Args &a, int ub) {
  __shared__ int all_ok;
  if (threadIdx.x == 0) all_ok = 1;
  __syncthreads();
  for (int i = threadIdx.x; i < a.P; i += NT)
    if (!head_accepts(a, ub, i)) atomicAnd(&all_ok, 0);
  __syncthreads();
  return all_ok != 0;
}

// Online (max, sum exp2) of slice `slice` of row r (W: elements per vector
// load), block-wide.  U (16-byte vectors per thread in flight per round)
// does not change the result: a thread folds its vectors in index order.
template <int NT, int W, int U>
__device__ __forceinline__ float2 slice_partial(const Args &a, int r, int slice) {
  const float c = a.c;
  const long long s0 = (long long)slice * a.Vw / a.S;
  const long long s1 = (long long)(slice + 1) * a.Vw / a.S;
  const float *row = row_ptr_u(a, r / a.rpb, r % a.rpb);
  float m = -INFINITY, s = 0.0f;
  if (W == 4) {
    // rounds of U vectors per thread, every load of a round issued before
    // the first use; in the last round a lane past the slice reloads its
    // last vector and folds -inf instead (exp2(-inf) = 0 and the max is
    // unchanged, so that is exactly nothing)
    const float4 *p4 = reinterpret_cast<const float4 *>(row);
    for (long long i0 = s0 + threadIdx.x; i0 < s1; i0 += U * NT) {
      float4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = ld_stream4(p4 + min(i0 + u * NT, s1 - 1));
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i0 + u * NT >= s1) v[u] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
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
  } else {
    for (long long i = s0 + threadIdx.x; i < s1; i += NT) {
      const float v = __builtin_nontemporal_load(row + i);
      if (v > m) {
        s *= __builtin_amdgcn_exp2f((m - v) * c);
        m = v;
      }
      const float ms = (m == -INFINITY) ? 0.0f : m;
      s += __builtin_amdgcn_exp2f((v - ms) * c);
    }
  }
  return block_ms<NT>(m, s, c);
}

// One work-group per (entry y of the row set, slice x): online
// (max, sum exp2) over the slice.
__device__ void mw_reset_share(const Args &a, long long wg, long long nwg);

// Threads of a statistics work-group (512 and 1024 measured 1% and 10%
// slower per C2 step).  A slice's partial depends on the fold order, which
// depends on the slice bounds (a function of the shape) and on the
// work-group size (which thread folds which vectors, the order of the block
// reduction): every statistics kernel uses kStatsNT threads, so the head,
// tail and one-pass statistics of a row combine identical partials.
constexpr int kStatsNT = 256;

template <int NT, int W>
__global__ __launch_bounds__(NT) void stats_kernel(Args a, int set) {
  static_assert(NT == kStatsNT, "every statistics pass folds a slice the same way");
  if (a.mw_reset && set != kRowsTail)
    mw_reset_share(a, (long long)blockIdx.y * gridDim.x + blockIdx.x, (long long)gridDim.x * gridDim.y);
  const int r = set_row(a, set, (int)blockIdx.x);
  if (r < 0) return;
  if (set == kRowsTail && !tail_needed<NT>(a, r / a.rpb)) return;
  const float2 out = slice_partial<NT, W, 4>(a, r, (int)blockIdx.y);
  if (threadIdx.x == 0) {
    a.part[(long long)r * a.S + blockIdx.y] = out;
    if (set == kRowsHead) {
      // the raw logit at this position's draft token, by the slice holding it
      const long long s0 = (long long)blockIdx.y * a.Vw / a.S;
      const long long s1 = (long long)(blockIdx.y + 1) * a.Vw / a.S;
      const int j = r % a.rpb, i = j <= a.K ? j : j - a.K - 1;
      const int t = min(max(a.tokens[(long long)(r / a.rpb) * a.K + i], 0), a.V - 1);
      if ((long long)t >= s0 * W && (long long)t < s1 * W)
        a.rawtok[r] = row_ptr_u(a, r / a.rpb, j)[t];
    }
  }
}

// Row groups the balanced tail pass can list in LDS.
constexpr int kTailMaxGroups = 4096;

// The tail pass, balanced over the device (16-byte loads; row groups <=
// kTailMaxGroups).  A grid of one work-group per (tail row, slice) leaves
// most work-groups with nothing to do (their sequence rejected a head
// position), and the CUs that happen to hold several busy ones pace the
// pass.  Here every work-group lists the groups that need their tail rows
// (one thread per group) and takes every gridDim.x-th (group, tail row,
// slice) item of that list, so every CU streams about the same bytes.  Each
// item's partial is the one stats_kernel computes for that (row, slice).
template <int NT>
__global__ __launch_bounds__(NT) void stats_tail_kernel(Args a) {
  static_assert(NT == kStatsNT, "every statistics pass folds a slice the same way");
  __shared__ int list[kTailMaxGroups];
  __shared__ int wcnt[NT / 64];
  __shared__ int base;
  const int groups = a.R / a.rpb;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) base = 0;
  __syncthreads();
  for (int g0 = 0; g0 < groups; g0 += NT) {
    const int ub = g0 + (int)threadIdx.x;
    bool need = ub < groups;
    if (need) need = head_all_accept(a, ub);
    const unsigned long long m = __ballot(need);
    if (lane == 0) wcnt[wave] = (int)__popcll(m);
    __syncthreads();
    int off = base;
    for (int w = 0; w < wave; ++w) off += wcnt[w];
    if (need) list[off + (int)__popcll(m & ((1ull << lane) - 1ull))] = ub;
    __syncthreads();
    if (threadIdx.x == 0)
      for (int w = 0; w < NT / 64; ++w) base += wcnt[w];
    __syncthreads();
  }
  const int K = a.K, P = a.P, per = 2 * (K - P) + 1;
  const long long total = (long long)base * per * a.S;
  for (long long k = blockIdx.x; k < total; k += gridDim.x) {
    const int ub = list[k / ((long long)per * a.S)];
    const int rem = (int)(k % ((long long)per * a.S));
    const int q = rem / a.S, slice = rem % a.S;
    const int r = ub * a.rpb + (q <= K - P ? P + q : K + 1 + P + (q - (K - P + 1)));
    const float2 out = slice_partial<NT, 4, 4>(a, r, slice);
    if (threadIdx.x == 0) a.part[(long long)r * a.S + slice] = out;
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

// One work-group per (row x, slice y).
template <int NT>
__global__ __launch_bounds__(NT) void argmax_kernel(Args a) {
  const int r = (int)blockIdx.x;
  if (r >= a.R) return;
  __shared__ float2 red[NT / 64];
  const int W = (int)(a.V / a.Vw);
  const long long e0 = (long long)blockIdx.y * a.Vw / a.S * W;
  const long long e1 = (long long)(blockIdx.y + 1) * a.Vw / a.S * W;
  const Dist d = make_dist_u(a, r / a.rpb, r % a.rpb);
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
    a.apart[(long long)r * a.S + blockIdx.y] = make_float2(v, __int_as_float(ix));
  }
}

__device__ int row_argmax(const Args &a, int r) {
  float v = -INFINITY;
  int ix = 0x7fffffff;
  for (int w = 0; w < a.S; ++w) {
    const float2 e = a.apart[(long long)r * a.S + w];
    am_merge(v, ix, e.x, __float_as_int(e.y));
  }
  return ix == 0x7fffffff ? 0 : ix;
}

// ---------------------------------------------------------------------------
// decide: one wave per sequence.
// ---------------------------------------------------------------------------

constexpr int kMaxK = 64;

struct DecideLds;
__device__ MwJob make_job(const Args &a, int b, int n, int kind, int row, int eos_acc, float u,
                         int extra = 0, float u2 = 0.0f, const DecideLds *L = nullptr);
__device__ void write_job(const Args &a, int b, const MwJob &j);

// The decision's inputs, gathered by a work-group of nt threads: the draft
// tokens and p(tok), q(tok) at every position with the statistics of every
// row of the sequence (or, greedy, the first argmax of every target row),
// and the sequence's uniforms.  One thread per row, so a row's partials and
// its value at the token are two rounds of loads for the whole gather.
struct DecideLds {
  float pt[kMaxK], qd[kMaxK];
  int tk[kMaxK], am[kMaxK + 1], ok[kMaxK];
  float2 st[2 * kMaxK + 1];  // (max, 1/S) of rows 0 .. 2K (logits input)
  float u[kMaxK + 2];
};

__device__ void decide_gather(const Args &a, int b, int tid, int nt, DecideLds &L) {
  const int K = a.K;
  if (a.mode == CFA_MODE_GREEDY) {
    for (int i = tid; i < K; i += nt) L.tk[i] = a.tokens[(long long)b * K + i];
    for (int i = tid; i <= K; i += nt) L.am[i] = row_argmax(a, (b / a.draws) * a.rpb + i);
    return;
  }
  // rows 0 .. K-1 target at a draft position, K the target's last row,
  // K+1 .. 2K draft
  for (int r = tid; r < 2 * K + 1; r += nt) {
    const int i = r <= K ? r : r - K - 1;
    const int traw = (r != K) ? a.tokens[(long long)b * K + i] : 0;
    const Dist d = make_dist(a, b, r);
    L.st[r] = make_float2(d.M, d.invS);
    if (r != K) {
      const int t = min(max(traw, 0), a.V - 1);  // never read outside the row
      const bool valid = traw == t;                // an id outside [0, V) is never accepted
      const float v = valid ? d(t) : 0.0f;
      if (r < K) {
        L.pt[i] = v;
        L.tk[i] = traw;
        L.ok[i] = valid ? 1 : 0;
      } else {
        L.qd[i] = v;
      }
    }
  }
  const int nu = min(a.ustride, kMaxK + 2);
  for (int i = tid; i < nu; i += nt) L.u[i] = a.U[(long long)b * a.ustride + i];
}

// cpp rules (speculative.cpp:66-97), one thread: the acceptance walk on the
// sequence's uniforms and the draw it still needs.
__device__ MwJob decide_cpp(const Args &a, int b, const DecideLds &L) {
  const int K = a.K;
  int n = 0, kind = kNone, row = -1, eos_acc = 0, draws = 0;
  float uf = 0.0f;
  for (int i = 0; i < K; ++i) {
    const float ratio = ratio_cpp(L.pt[i], L.qd[i]);
    const float r = L.u[draws++];
    if (L.ok[i] && r <= ratio) {
      ++n;
      if (L.tk[i] == a.eos) {
        eos_acc = 1;
        break;
      }
    } else {
      kind = kResid;
      row = i;
      uf = L.u[draws++];
      break;
    }
  }
  if (!eos_acc && kind == kNone) {
    kind = kPlain;
    row = K;
    uf = L.u[draws++];
  }
  return make_job(a, b, n, kind, row, eos_acc, uf, 0, 0.0f, &L);
}

// One work-group per sequence.  cpp mode runs this only where the exact
// draw is not needed (the mw sums kernel decides otherwise); python mode
// records n_b for plan_kernel; greedy writes the final outputs.
__global__ __launch_bounds__(64) void decide_kernel(Args a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  __shared__ DecideLds L;
  const int K = a.K;
  decide_gather(a, b, lane, 64, L);
  __syncthreads();
  if (lane != 0) return;
  if (a.mode == CFA_MODE_CPP) {
    write_job(a, b, decide_cpp(a, b, L));
    return;
  }
  int n = 0, eos_acc = 0;
  if (a.mode == CFA_MODE_PYTHON) {
    n = K;
    for (int i = 0; i < K; ++i)
      if (!(L.u[i] < ratio_py(L.pt[i], L.qd[i]))) {
        n = i;
        break;
      }
    a.dec[b] = make_int4(n, kNone, -1, 0);
    a.ufin[b] = L.u[K];
    return;
  }
  // greedy: outputs are final here
  int fin = -1;
  for (int i = 0; i < K; ++i) {
    if (L.tk[i] == L.am[i]) {
      ++n;
      if (L.tk[i] == a.eos) {
        eos_acc = 1;
        fin = a.eos;
        break;
      }
    } else {
      fin = L.am[i];
      break;
    }
  }
  if (!eos_acc && n == K) fin = L.am[K];
  int32_t *ot = a.out_tokens + (long long)b * (K + 1);
  for (int j = 0; j <= K; ++j) ot[j] = (j < n) ? L.tk[j] : -1;
  if (!eos_acc) ot[n] = fin;
  a.out_accept_len[b] = n;
  a.out_final[b] = fin;
  a.out_eos[b] = (eos_acc || fin == a.eos) ? 1 : 0;
  a.out_num_emitted[b] = eos_acc ? n : n + 1;
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

// The top_k-th largest probability (ties kept): the least v with
// #{p_i > v} < top_k, found by bisection on the fp32 bits.
template <int NT>
__device__ float topk_threshold(const Dist &t, int V, int top_k, double *red) {
  uint32_t lo = 0, hi = 0x7f800000u;
  while (hi - lo > 1) {
    const uint32_t mid = lo + (hi - lo) / 2;
    const float tau = u2f(mid);
    double cnt = 0.0;
    for (int i = threadIdx.x; i < V; i += NT) cnt += (t(i) > tau) ? 1.0 : 0.0;
    if (block_sum_f64<NT>(cnt, red) < (double)top_k)
      hi = mid;
    else
      lo = mid;
  }
  return u2f(hi);
}

// ---------------------------------------------------------------------------
// plan: the draw each sequence still needs.  Python mode applies the batch
// lock-step rule n = min_b n_b of speculative.py:166 here; cpp mode's draws
// are per sequence, so decide writes them directly.
// ---------------------------------------------------------------------------

// Python-mode draws take the first index whose sequential prefix sum
// EXCEEDS u (so u = 0 never selects a zero-weight entry, as torch.multinomial
// never does); the inverse-CDF walks test `r <= prefix`, and for floats
// u < x <=> succ(u) <= x.  The floor FLT_MIN keeps r out of the denormals.
__device__ __forceinline__ float py_threshold(float u) {
  // for finite u >= 0 the next float up is the next bit pattern
  const float s = (u >= 0.0f && u < INFINITY) ? __uint_as_float(__float_as_uint(u) + 1u) : u;
  return fmaxf(s, 1.17549435e-38f);
}

// The job of sequence b: its draw (n, kind, row, eos_acc, threshold u; a
// python-mode bonus after the resample when extra) and the statistics of the
// draw's rows, once for every kernel that reads them.
__device__ MwJob make_job(const Args &a, int b, int n, int kind, int row, int eos_acc, float u,
                         int extra, float u2, const DecideLds *L) {
  const int K = a.K;
  MwJob j;
  j.n = n;
  j.kind = kind;
  j.row = row;
  j.eos_acc = eos_acc;
  j.u = u;
  j.extra = extra;
  j.u2 = u2;
  j.pad = 0;
  j.tM = j.dM = 0.0f;
  j.tInvS = j.dInvS = 1.0f;
  if (a.logits && (j.kind == kResid || j.kind == kPlain)) {
    // the rows' statistics, from the gather when it has them
    const float2 ts = L ? L->st[j.row] : row_stat(a, (b / a.draws) * a.rpb + j.row);
    j.tM = ts.x;
    j.tInvS = ts.y;
    if (j.kind == kResid) {
      const float2 ds = L ? L->st[K + 1 + j.row] : row_stat(a, (b / a.draws) * a.rpb + K + 1 + j.row);
      j.dM = ds.x;
      j.dInvS = ds.y;
    }
  }
  return j;
}

// Store the job and reset the walk state of b.
__device__ void write_job(const Args &a, int b, const MwJob &j) {
  a.jobs[b] = j;
  a.res[b] = MwRes{0.0f, 0, -1, -1};
  a.badcnt[b] = 0;
  a.badcnt[a.B + b] = 0;
}

// Python mode only (cpp mode decides each sequence's draw by itself).
__global__ __launch_bounds__(256) void plan_kernel(Args a) {
  __shared__ int nmin;
  const int K = a.K;
  if (threadIdx.x == 0) nmin = K;
  __syncthreads();
  int local = K;
  for (int q = threadIdx.x; q < a.B; q += blockDim.x) local = min(local, a.dec[q].x);
  atomicMin(&nmin, local);
  __syncthreads();
  // A rejection at the last position (n = K - 1) brings the reference's
  // num_accepted to K, so its `num_accepted == self.k` branch
  // (speculative.py:188-195) appends a bonus draw after the resample.
  const int extra = (K > 0 && nmin == K - 1) ? 1 : 0;
  for (int b = threadIdx.x; b < a.B; b += blockDim.x) {
    const float u2 = extra ? py_threshold(a.U[(long long)b * a.ustride + K + 1]) : 0.0f;
    write_job(a, b, make_job(a, b, nmin, (nmin < K) ? kResid : kPyBonus, (nmin < K) ? nmin : K, 0,
                             py_threshold(a.ufin[b]), extra, u2));
  }
}

// ---------------------------------------------------------------------------
// Exact draw over all work-groups ("mw").  A row is cut into chunks of 1024
// elements (64 tiles of 16, one wave per chunk).  For each drawing sequence:
//   sums     approximate fp32 chunk sums of the residual and of the target
//            row, used only to guess regions;
//   records  per pass: every tile quantised in its guessed region
//            (seqsum.hpp); per chunk, the composed function of the tiles
//            before its first break (a tile straddling a region boundary, or
//            a region change), the break, and the function of the tiles
//            after it; tiles that will need a serial replay are cached;
//   walk     per pass, one wave: chunk 0, where the running value is small
//            and crosses a binade every doubling, is walked tile by tile
//            from its records (the records also store all its values, so the
//            straddling tiles replay from LDS); later chunks apply their
//            functions from the exact running value, and a chunk with a
//            break costs a check, the break tile's serial replay and a second
//            check.  Any check that fails (a wrong guess, a second break, a
//            CDF hit inside a run) falls back to the tile-level walk of
//            seq::walk.
// Two launches: mw_first_kernel (the decision, the sums and the sum pass's
// records) and mw_tail_kernel (the sum pass's walk, the CDF pass's records
// and walk, job by job).
// Pass 0 sums max(0, t - d) (speculative.cpp:30-35); pass 1 searches the
// inverse CDF of max(0, t - d) / S, or of t for a bonus draw or the
// sum <= 1e-6 fallback (speculative.cpp:11-24, 37-45, 97).
// ---------------------------------------------------------------------------

enum MwPass : int { kPassSum = 0, kPassCdf = 1 };
enum MwStatus : int { kChunkOk = 0, kChunkTiles = 1, kChunkSkipped = 2 };

// The element function of a (job, pass): 0 max(0,t-d), 1 max(0,t-d)/S, 2 t.
struct MwElem {
  Dist t, d;
  int fn;
  float S;
  __device__ __forceinline__ float eval(float tv, float dv) const {
    if (fn == 2) return t.eval(tv);
    const float x = relu_ref(t.eval(tv) - d.eval(dv));
    return fn == 1 ? x / S : x;
  }
};

__device__ __forceinline__ bool mw_active(const MwJob &j, int pass) {
  return pass == kPassSum ? j.kind == kResid : (j.kind == kResid || j.kind == kPlain);
}

// The element function of (job b, pass); `r` holds the sum pass's result
// (S, fallback) for the CDF pass.
__device__ __forceinline__ MwElem mw_elem_r(const Args &a, int b, const MwJob &j, int pass, const MwRes &r) {
  MwElem e;
  e.t.p = row_ptr(a, b, j.row);
  e.t.c = a.c;
  e.t.logits = a.logits;
  e.t.M = j.tM;
  e.t.invS = j.tInvS;
  e.d = e.t;
  e.S = 1.0f;
  if (j.kind == kResid) {
    e.d.p = row_ptr(a, b, a.K + 1 + j.row);
    e.d.M = j.dM;
    e.d.invS = j.dInvS;
  }
  if (pass == kPassSum) {
    e.fn = 0;
  } else {
    e.fn = (j.kind == kResid && !r.fallback) ? 1 : 2;
    e.S = r.S;
  }
  return e;
}

__device__ __forceinline__ MwElem mw_elem(const Args &a, int b, const MwJob &j, int pass) {
  return mw_elem_r(a, b, j, pass, pass == kPassSum ? MwRes{} : a.res[b]);
}

// Raw values of 16 consecutive elements starting at i0 (zero past V).
__device__ __forceinline__ void mw_load16(const Args &a, const float *p, long long i0, float *v) {
  if (a.vec && i0 + kMwTile <= a.V) {
    const float4 *p4 = reinterpret_cast<const float4 *>(p + i0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 q = p4[k];
      v[4 * k] = q.x;
      v[4 * k + 1] = q.y;
      v[4 * k + 2] = q.z;
      v[4 * k + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kMwTile; ++k) v[k] = (i0 + k < a.V) ? p[i0 + k] : 0.0f;
  }
}

// Raw target and draft values of tile `tile` (the draft only when the
// element function reads it).
__device__ __forceinline__ void mw_tile_raw(const Args &a, const MwElem &e, long long tile,
                                            float *tv, float *dv) {
  const long long i0 = tile * kMwTile;
  mw_load16(a, e.t.p, i0, tv);
  if (e.fn != 2) mw_load16(a, e.d.p, i0, dv);
}

// Evaluated elements of tile `tile` from its raw values (zero past V).
__device__ __forceinline__ void mw_tile_eval(const Args &a, const MwElem &e, long long tile,
                                             const float *tv, const float *dv, float *x) {
  const long long i0 = tile * kMwTile;
#pragma unroll
  for (int k = 0; k < kMwTile; ++k) x[k] = (i0 + k < a.V) ? e.eval(tv[k], e.fn != 2 ? dv[k] : 0.0f) : 0.0f;
}

// Evaluated elements of tile `tile` of a row (zero past V).
__device__ __forceinline__ void mw_tile_values(const Args &a, const MwElem &e, long long tile,
                                               float *x) {
  float tv[kMwTile], dv[kMwTile];
  mw_tile_raw(a, e, tile, tv, dv);
  mw_tile_eval(a, e, tile, tv, dv, x);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Approximate running value at the start of chunk c: the chunk sums before
// it, in a fixed order (one wave).
__device__ float mw_entry_prefix(const float *csum, int c) {
  const int lane = threadIdx.x & 63;
  float acc = 0.0f;
  for (int base = 0; base < c; base += 64) {
    float v = (base + lane < c) ? csum[base + lane] : 0.0f;
    acc += wave_sum_f32(v);
  }
  return acc;
}

// Composition of the functions of the lanes where `in` holds (lane order).
__device__ __forceinline__ seq::Inc wave_compose_where(bool in, seq::Inc f) {
  using namespace seq;
  const Inc v = in ? f : inc_identity();
  const Inc tot = (__ballot(v.e != v.o) == 0ull) ? Inc{wave_incl_add_u32(v.e), 0u}
                                                 : wave_incl_compose(v);
  if (__ballot(v.e != v.o) == 0ull) {
    const uint32_t t = lane_bcast(tot.e, 63);
    return Inc{t, t};
  }
  return Inc{lane_bcast(tot.e, 63), lane_bcast(tot.o, 63)};
}

// A CDF search ends before any chunk whose approximate entry value E0 is
// surely past u; such a chunk gets a "skipped" record and no loads.
__device__ __forceinline__ bool mw_skip(int pass, const MwJob &j, float E0) {
  return pass == kPassCdf && E0 * (1.0f - 1.0f / 64.0f) > j.u;
}

__device__ __forceinline__ void mw_write_skipped(const Args &a, long long rowrec, int c) {
  if ((threadIdx.x & 63) == 0) {
    MwChunk r{};
    r.status = kChunkSkipped;
    a.crec[rowrec * a.NC + c] = r;
  }
}

// Records of chunk c of job b for one pass, by one wave (lane = tile in the
// chunk), from the chunk's approximate entry value E0 (on the pass's scale)
// and the lane's 16 evaluated elements.  For chunk 0, tr_lds / xs_lds (if
// given) also receive its tile records and values in LDS, for a walk of
// chunk 0 by the same wave.
__device__ __forceinline__ void mw_records_chunk(const Args &a, int b, int c, int pass,
                                                 const MwJob &j, float E0, const float *x,
                                                 MwRec *tr_lds = nullptr, float *xs_lds = nullptr) {
  using namespace seq;
  const int lane = threadIdx.x & 63;
  const long long rowrec = ((long long)pass * a.B + b);
  MwChunk *crec = a.crec + rowrec * a.NC;
  MwRec *trec = a.trec + rowrec * a.NC * kMwChunkTiles;
  const long long tile = (long long)c * kMwChunkTiles + lane;
  float A = 0.0f;
#pragma unroll
  for (int k = 0; k < kMwTile; ++k) A += x[k];
  const float incl = wave_incl_scan_f32(A);
  const float E = E0 + (incl - A);
  int r_lo = region_of(E * (1.0f - kDelta));
  const int r_hi = region_of((E + A) * (1.0f + kDelta));
  bool ok = (r_lo == r_hi);
  Inc f{kBad, kBad};
  if (A == 0.0f) {
    ok = true;
    r_lo = kAnyRegion;
    f = inc_identity();
  } else if (ok) {
    uint32_t I;
    if (quantize_tile_fast(x, kMwTile, r_lo, I))
      f = Inc{I, I};
    else
      quantize_tile(x, kMwTile, r_lo, f.e, f.o);
    ok = (f.e <= kUnitsTop) && (f.o <= kUnitsTop);
    if (!ok) f = Inc{kBad, kBad};
  }
  const MwRec rec_t{f.e, f.o, ok ? r_lo : kAnyRegion, ok ? 0 : 1};
  trec[tile] = rec_t;
  if (c == 0) {  // chunk 0 is walked tile by tile: all its values go to the walk
    float4 *dst = reinterpret_cast<float4 *>(a.x0 + rowrec * kMwChunk + lane * kMwTile);
#pragma unroll
    for (int k = 0; k < kMwTile; k += 4) dst[k / 4] = make_float4(x[k], x[k + 1], x[k + 2], x[k + 3]);
    if (tr_lds != nullptr) {
      tr_lds[lane] = rec_t;
      float4 *dl = reinterpret_cast<float4 *>(xs_lds + lane * kMwTile);
#pragma unroll
      for (int k = 0; k < kMwTile; k += 4) dl[k / 4] = make_float4(x[k], x[k + 1], x[k + 2], x[k + 3]);
    }
    return;
  }
  // Cache the values of the tiles the walk will probably replay serially: a
  // straddling tile (!ok), a tile within kMwNear of a binade (the exact
  // running value can sit on the other side of the boundary from the
  // approximate one), and in the CDF pass a tile whose approximate range
  // holds u (where the search ends).  One slot reservation per wave.
  const bool nearb = A != 0.0f && region_of(E * (1.0f - kMwNear)) != region_of((E + A) * (1.0f + kMwNear));
  const bool hitc = pass == kPassCdf && A != 0.0f && E * (1.0f - kMwNear) <= j.u &&
                    j.u <= (E + A) * (1.0f + kMwNear);
  const bool keep = !ok || nearb || hitc;
  const unsigned long long keepm = __ballot(keep);
  if (keepm) {
    const int first = (int)__builtin_ctzll(keepm);
    int base = 0;
    if (lane == first) base = atomicAdd(&a.badcnt[rowrec], (int)__popcll(keepm));
    base = (int)lane_bcast((uint32_t)base, first);
    const int slot = base + (int)__popcll(keepm & ((1ull << lane) - 1ull));
    if (keep && slot < kMwMaxBad) {
      MwBad *dst = a.bad + rowrec * kMwMaxBad + slot;
      dst->tile = (int)tile;
#pragma unroll
      for (int k = 0; k < kMwTile; ++k) dst->x[k] = x[k];
    }
  }
  // chunk structure: run 0, an optional break, run 1
  const bool real = ok && r_lo != kAnyRegion;
  const unsigned long long realm = __ballot(real);
  const int r_first = realm ? (int)lane_bcast((uint32_t)r_lo, (int)__builtin_ctzll(realm)) : kAnyRegion;
  const unsigned long long brkm = __ballot(!ok || (real && r_lo != r_first));
  MwChunk rec{};
  rec.status = kChunkOk;
  rec.near = keepm != 0ull;
  if (brkm == 0ull) {
    const Inc F = wave_compose_where(true, f);
    rec.e0 = F.e;
    rec.o0 = F.o;
    rec.reg0 = r_first;
    rec.brk = -1;
  } else {
    const int k = (int)__builtin_ctzll(brkm);
    const bool kbad = ((__ballot(!ok) >> k) & 1ull) != 0ull;
    const int s1 = kbad ? k + 1 : k;
    const unsigned long long before = (k == 0) ? 0ull : (~0ull >> (64 - k));
    const Inc F0 = wave_compose_where(lane < k, f);
    const bool in1 = lane >= s1;
    const unsigned long long real1 = realm & ~((s1 >= 64) ? ~0ull : ((1ull << s1) - 1ull));
    const int r1 = real1 ? (int)lane_bcast((uint32_t)r_lo, (int)__builtin_ctzll(real1)) : kAnyRegion;
    const bool bad1 = in1 && (!ok || (real && r_lo != r1));
    const Inc F1 = wave_compose_where(in1, f);
    rec.e0 = F0.e;
    rec.o0 = F0.o;
    rec.reg0 = (realm & before) ? r_first : kAnyRegion;
    rec.brk = k;
    rec.brk_serial = kbad ? 1 : 0;
    rec.e1 = F1.e;
    rec.o1 = F1.o;
    rec.reg1 = r1;
    if (__ballot(bad1) != 0ull) rec.status = kChunkTiles;
  }
  if (rec.status == kChunkTiles) rec.near = 1;
  if (lane == 0) crec[c] = rec;
}

// Zeroes this work-group's share (work-group wg of nwg) of the first exact
// pass's look-back words, of both passes' cache counters and of the tail
// kernel's synchronisation words.  The first kernel of every call that draws
// exactly runs this, so nothing in the workspace has to start at zero.
__device__ void mw_reset_share(const Args &a, long long wg, long long nwg) {
  const long long nt = blockDim.x, i0 = wg * nt + threadIdx.x, step = nwg * nt;
  for (long long i = i0; i < (long long)a.B * a.NC; i += step) a.flags[i] = 0ull;
  for (long long i = i0; i < 2LL * a.B; i += step) {
    a.badcnt[i] = 0;
    a.tsync[i] = 0ull;
  }
}

__global__ __launch_bounds__(256) void mw_reset_kernel(Args a) {
  mw_reset_share(a, blockIdx.x, gridDim.x);
}

// Look-back words: status in bits 62-63 (0 none, 1 the chunk's own sum,
// 2 the inclusive prefix through the chunk), the fp32 value in bits 0-31.
// They cross work-groups (and XCDs, whose L2s are not coherent with each
// other) as agent-scope atomic stores and loads.
constexpr unsigned long long kLbAgg = 1ull << 62, kLbIncl = 2ull << 62;
constexpr long kLbSpins = 1l << 16;  // a bounded wait: the value only steers region guesses

__device__ __forceinline__ void lb_store(unsigned long long *p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long lb_load(unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Approximate running value at the start of chunk c of job b by decoupled
// look-back over the chunks before it (one wave): publish the chunk's own
// sum, add the predecessors' published sums back to the nearest inclusive
// prefix, publish the inclusive prefix.  Work-groups start in block order, so
// a predecessor is already running or done; still, every wait is bounded,
// and one that runs out keeps what it has -- the value only guides the
// region guesses of the records, which the walk checks against the exact
// running value, so a poor value costs time, never correctness.
__device__ float mw_lookback(const Args &a, int b, int c, float own) {
  const int lane = threadIdx.x & 63;
  unsigned long long *fl = a.flags + (long long)b * a.NC;
  if (c == 0) {
    if (lane == 0) lb_store(fl, kLbIncl | f2u(own));
    return 0.0f;
  }
  if (lane == 0) lb_store(fl + c, kLbAgg | f2u(own));
  float pre = 0.0f;
  long spins = 0;
  for (int j = c - 1; j >= 0; j -= 64) {
    const int idx = j - lane;  // lanes look at chunks j, j - 1, ..., j - 63
    unsigned long long w = 0;
    int stop = 63;      // lanes 0 .. stop add their value
    bool done = false;  // an inclusive prefix (or a wait that ran out) ends the look-back
    for (;;) {
      w = idx >= 0 ? lb_load(fl + idx) : kLbIncl;  // before chunk 0: an inclusive zero
      const unsigned long long ready = __ballot((w >> 62) != 0ull);
      const unsigned long long incl = __ballot((w >> 62) == 2ull);
      const int fi = incl ? (int)__builtin_ctzll(incl) : 64;
      const int fw = ~ready ? (int)__builtin_ctzll(~ready) : 64;
      if (fi < fw) {  // every chunk down to the nearest inclusive prefix has published
        stop = fi;
        done = true;
        break;
      }
      if (fw == 64) break;  // 64 own sums: go on below them
      if (++spins > kLbSpins) {  // keep the chunks before the first silent one
        stop = fw - 1;
        done = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    pre += wave_sum_f32(lane <= stop && idx >= 0 ? u2f((uint32_t)w) : 0.0f);
    if (done) break;
  }
  if (lane == 0) lb_store(fl + c, kLbIncl | f2u(pre + own));
  return pre;
}

// Orders one wave's LDS accesses (a wave's LDS operations complete in issue
// order, so this only keeps the compiler from moving accesses across it).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Serial replay of a tile's 16 values x from s (CDF: first hit index, the
// first i with r <= s_i, else -1).  The running value never decreases
// (x >= 0), so the hit is searched only in a tile whose last partial sum
// reaches r.
__device__ __forceinline__ long long mw_replay16(const float *x, long long i0, float &s, bool cdf,
                                                 float r) {
  float ps[kMwTile];
  float acc = s;
#pragma unroll
  for (int k = 0; k < kMwTile; ++k) {
    acc = acc + x[k];
    ps[k] = acc;
  }
  if (cdf && r <= acc) {
    // static indices only: a dynamically indexed ps[] would live in scratch
    int k = kMwTile - 1;
    float sk = ps[kMwTile - 1];
#pragma unroll
    for (int q = kMwTile - 2; q >= 0; --q) {
      const bool h = r <= ps[q];
      k = h ? q : k;
      sk = h ? ps[q] : sk;
    }
    s = sk;
    return i0 + k;
  }
  s = acc;
  return -1;
}

// Chunk 0 of a row, walked by one wave from 0 with its values xs[kMwChunk]
// and tile records tr[64] in LDS: the first kMwSerialTiles tiles replayed
// serially (the small running value doubles every few elements there: 1, 2,
// 4, ... 32 for a flat row), then runs of tiles applied from their records,
// the tiles straddling a binade replayed serially.  Touches no global
// memory.  Returns the CDF hit (or -1) and leaves the running value in s.
__device__ __forceinline__ long long mw_walk_chunk0(const float *xs, const MwRec *tr, bool cdf, float r,
                                                    float &s) {
  using namespace seq;
  s = 0.0f;
  long long found = -1;
  {
    const float4 *h4 = reinterpret_cast<const float4 *>(xs);
    float xh[kMwSerialTiles * kMwTile];
#pragma unroll
    for (int k = 0; k < kMwSerialTiles * kMwTile / 4; ++k) {
      const float4 q = h4[k];
      xh[4 * k] = q.x;
      xh[4 * k + 1] = q.y;
      xh[4 * k + 2] = q.z;
      xh[4 * k + 3] = q.w;
    }
#pragma unroll
    for (int t = 0; t < kMwSerialTiles; ++t)
      if (found < 0) found = mw_replay16(xh + t * kMwTile, (long long)t * kMwTile, s, cdf, r);
  }
  if (found < 0) {
    auto item0 = [&](int i, int &reg) -> Inc {
      const MwRec q = tr[kMwSerialTiles + i];
      reg = q.reg;
      return q.pad ? Inc{kBad, kBad} : Inc{q.e, q.o};
    };
    auto desc0 = [&](int i0, float &s2) -> long long {
      const int i = kMwSerialTiles + i0;
      const float4 *x4 = reinterpret_cast<const float4 *>(xs + i * kMwTile);
      float x[kMwTile];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 q = x4[k];
        x[4 * k] = q.x;
        x[4 * k + 1] = q.y;
        x[4 * k + 2] = q.z;
        x[4 * k + 3] = q.w;
      }
      return mw_replay16(x, (long long)i * kMwTile, s2, cdf, r);
    };
    found = walk(kMwChunkTiles - kMwSerialTiles, s, cdf, r, item0, desc0);
  }
  return found;
}

// Chunks per wave of mw_first_kernel: two, so that the launch has B * NC / 2
// waves (4032 at C2) and every wave is resident from the start -- with one
// chunk per wave (8064 waves, against about 7 resident per SIMD) the last
// eight sequences' work-groups started 12 us late, after the first ones
// ended (36.1 -> 29.4 us at C2).
constexpr int kMwCPW = 2;
constexpr int kMwChunksPerWG = (kMwNT / 64) * kMwCPW;

// The first exact pass, with the chunk sums: each wave takes chunks c0 and
// c0 + 1 (c0 = 2 (4 blockIdx.x + wave)) of job blockIdx.y, lane = tile in the
// chunk.  With `decide` (cpp rules) every work-group first takes sequence
// b's decision itself (decide_cpp: the same inputs, so the same job
// everywhere) and the first one stores it.  Every active job stores its
// chunk sums of t (the CDF pass of a plain draw, or of the fallback, starts
// from them); a residual job also stores those of max(0, t - d), finds its
// chunks' entry values by look-back (both chunks' own sums published first),
// and writes the sum pass's records (mw_records_chunk).  The wave holding
// chunk 0 then walks it (the walk's slowest chunk: its small running value
// crosses a binade every few elements) and stores the exact running value
// after it, so the sum pass's walk starts at chunk 1.
__global__ __launch_bounds__(kMwNT) void mw_first_kernel(Args a, int decide) {
  __shared__ __align__(16) float xs0[kMwChunk];  // chunk 0's values and tile records
  __shared__ MwRec tr0[kMwChunkTiles];
  const int b = blockIdx.y, lane = threadIdx.x & 63;
  const int c0 = kMwCPW * (blockIdx.x * (kMwNT / 64) + (threadIdx.x >> 6));
  MwJob j;
  if (decide) {
    __shared__ DecideLds L;
    __shared__ MwJob sj;
    decide_gather(a, b, threadIdx.x, kMwNT, L);
    __syncthreads();
    if (threadIdx.x == 0) {
      sj = decide_cpp(a, b, L);
      if (blockIdx.x == 0) {  // the cache counters were zeroed by an earlier kernel
        a.jobs[b] = sj;
        a.res[b] = MwRes{0.0f, 0, -1, -1};
      }
    }
    __syncthreads();
    j = sj;
  } else {
    j = a.jobs[b];
  }
  if (j.kind != kResid && j.kind != kPlain) return;
  if (c0 >= a.NC) return;
  const bool two = c0 + 1 < a.NC;
  const bool resid = j.kind == kResid;
  const MwElem e = mw_elem(a, b, j, kPassSum);
  float tv[kMwCPW][kMwTile], dv[kMwCPW][kMwTile], x[kMwCPW][kMwTile];
  // both chunks' loads before any use
#pragma unroll
  for (int h = 0; h < kMwCPW; ++h) {
    const long long i0 = ((long long)(c0 + (two ? h : 0)) * kMwChunkTiles + lane) * kMwTile;
    mw_load16(a, e.t.p, i0, tv[h]);
    if (resid) mw_load16(a, e.d.p, i0, dv[h]);
  }
  float sx[kMwCPW];
#pragma unroll
  for (int h = 0; h < kMwCPW; ++h) {
    const long long i0 = ((long long)(c0 + h) * kMwChunkTiles + lane) * kMwTile;
    float st = 0.0f, sxh = 0.0f;
#pragma unroll
    for (int k = 0; k < kMwTile; ++k) {
      x[h][k] = 0.0f;
      if (i0 + k < a.V) {
        const float tp = e.t.eval(tv[h][k]);
        st += tp;
        if (resid) {
          x[h][k] = relu_ref(tp - e.d.eval(dv[h][k]));
          sxh += x[h][k];
        }
      }
    }
    st = wave_sum_f32(st);
    sx[h] = wave_sum_f32(sxh);
    if (lane == 0 && (h == 0 || two)) {
      a.csum_t[(long long)b * a.NC + c0 + h] = st;
      a.csum_x[(long long)b * a.NC + c0 + h] = sx[h];
    }
  }
  if (!resid) return;
  unsigned long long *fl = a.flags + (long long)b * a.NC;
  if (two && lane == 0) lb_store(fl + c0 + 1, kLbAgg | f2u(sx[1]));  // before c0's look-back
  const float E0 = mw_lookback(a, b, c0, sx[0]);
  const bool walk0 = c0 == 0;  // wave-uniform
  mw_records_chunk(a, b, c0, kPassSum, j, E0, x[0], walk0 ? tr0 : nullptr, walk0 ? xs0 : nullptr);
  if (two) {
    const float E1 = E0 + sx[0];
    if (lane == 0) lb_store(fl + c0 + 1, kLbIncl | f2u(E1 + sx[1]));
    mw_records_chunk(a, b, c0 + 1, kPassSum, j, E1, x[1]);
  }
  if (walk0) {
    wave_sync();
    float s0;
    mw_walk_chunk0(xs0, tr0, false, 0.0f, s0);
    if (lane == 0) a.s0[b] = s0;
  }
}

constexpr int kMwWin = 256;  // chunk records staged in LDS at a time

__device__ __forceinline__ void finish_one(const Args &a, int b, const MwJob &j, int idx,
                                           int idx2 = -1);

// Last index of positive weight of a (job, pass) row, V - 1 if none; one
// wave scans down from the end (python mode's rare fallback draw).
__device__ long long mw_last_positive(const Args &a, const MwElem &e) {
  const int lane = threadIdx.x & 63;
  for (long long base = ((long long)(a.V - 1) / 64) * 64; base >= 0; base -= 64) {
    const long long i = base + lane;
    bool pos = false;
    if (i < a.V) pos = e.eval(e.t.load(i), e.fn != 2 ? e.d.load(i) : 0.0f) > 0.0f;
    const unsigned long long m = __ballot(pos);
    if (m) return base + 63 - __builtin_clzll(m);
  }
  return a.V - 1;
}

// LDS of one walk.
struct MwWalkLds {
  MwChunk cr[kMwWin];
  MwRec tr[kMwChunkTiles];
  MwRec pft[kMwPf][kMwChunkTiles];  // tile records of the prefetched chunks
  MwBad bad[kMwMaxBad];
  alignas(16) float xs[kMwChunk];
};


// The exact walk of job b's row for one pass, by the calling wave alone: it
// synchronises only itself, so the other waves of its work-group can wait at
// a barrier meanwhile.  Writes the pass's result (sum pass: S and the
// fallback flag; CDF pass: the drawn index, and the outputs in cpp mode) and
// returns the final running value.  use_cache = false ignores the cached
// serial tiles (another work-group may still be filling a slot); the walk
// then reads those tiles' values from the row.  pre0: chunk 0 was already
// walked (mw_walk_chunk0), ending at running value s0 with hit found0.
__device__ __forceinline__ float mw_walk(const Args &a, int b, int pass, const MwJob &j,
                                         const MwElem &e, MwWalkLds &L, bool use_cache = true,
                                         bool pre0 = false, float s0 = 0.0f, long long found0 = -1) {
  using namespace seq;
  MwChunk *cr = L.cr;
  MwRec *tr = L.tr;
  MwRec(&pft)[kMwPf][kMwChunkTiles] = L.pft;
  MwBad *bad = L.bad;
  float *xs = L.xs;
  const int lane = threadIdx.x & 63;
  const long long rowrec = ((long long)pass * a.B + b);
  const MwChunk *crec = a.crec + rowrec * a.NC;
  const MwRec *trec = a.trec + rowrec * a.NC * kMwChunkTiles;

  // One round of loads before the first wait: chunk 0's values and tile
  // records (unless chunk 0 was walked already), the first window of chunk
  // records, every cache slot (all written by the records for active jobs;
  // in-bounds, unused otherwise) and the cache count.
  if (!pre0) {
    const float4 *src = reinterpret_cast<const float4 *>(a.x0 + rowrec * kMwChunk + lane * kMwTile);
    float4 *dst = reinterpret_cast<float4 *>(xs + lane * kMwTile);
#pragma unroll
    for (int k = 0; k < kMwTile / 4; ++k) dst[k] = src[k];
    tr[lane] = trec[lane];
  }
  for (int c = 1 + lane; c < min(a.NC, 1 + kMwWin); c += 64) cr[c - 1] = crec[c];
  static_assert(kMwMaxBad <= 64, "one cache slot per lane");
  bad[lane] = a.bad[rowrec * kMwMaxBad + lane];
  const int nbad = use_cache ? min(a.badcnt[rowrec], kMwMaxBad) : 0;
  wave_sync();
  const bool cdf = (pass == kPassCdf);
  const float r = j.u;

  // The first kMwPf chunks of the first window that the records
  // flagged `near`: lane p < npf holds the p-th one's index.  Their tile
  // records travel straight to LDS during the chunk-0 walk (which touches
  // no global memory), so a tile-level walk there costs no round trip.
  int pfc = -1, npf = 0;
  {
    const int cnt0 = min(kMwWin, a.NC - 1);
    for (int base = 0; base < cnt0 && npf < kMwPf; base += 64) {
      const int i = base + lane;
      unsigned long long m = __ballot(i < cnt0 && cr[i].near != 0);
      while (m != 0ull && npf < kMwPf) {
        const int k = (int)__builtin_ctzll(m);
        if (lane == npf) pfc = 1 + base + k;
        ++npf;
        m &= m - 1ull;
      }
    }
  }
  for (int p = 0; p < npf; ++p) {
    const int cp = (int)lane_bcast((uint32_t)pfc, p);
    dma16(trec + (long long)cp * kMwChunkTiles + lane, (CFA_LDS void *)pft[p]);
  }

  auto replay16 = [&](const float *x, long long i0, float &s) -> long long {
    return mw_replay16(x, i0, s, cdf, r);
  };
  // values of tile `tile`: the cache when the records stored them
  auto serial = [&](long long tile, float &s) -> long long {
    const int q = lane < nbad ? lane : 0;
    const unsigned long long m = __ballot(lane < nbad && bad[q].tile == (int)tile);
    float x[kMwTile];
    if (m) {
      const MwBad &bt = bad[__builtin_ctzll(m)];
#pragma unroll
      for (int k = 0; k < kMwTile; ++k) x[k] = bt.x[k];
    } else {
      mw_tile_values(a, e, tile, x);
    }
    return replay16(x, tile * kMwTile, s);
  };

  // chunk 0, unless it was walked already
  float s = s0;
  long long found = found0;
  if (!pre0) found = mw_walk_chunk0(xs, tr, cdf, r, s);
  wait_vmcnt<0>();
  wave_sync();

  // tile-level walk of chunk c from its tile t0 (records from the prefetch
  // table, else from memory)
  auto tile_walk = [&](int c, int t0, float &ss) -> long long {
    const unsigned long long pm = __ballot(lane < npf && pfc == c);
    const MwRec *trs = tr;
    if (pm != 0ull) {
      trs = pft[__builtin_ctzll(pm)];
    } else {
      wave_sync();
      tr[lane] = trec[(long long)c * kMwChunkTiles + lane];
      wave_sync();
    }
    auto tile_item = [&](int i, int &reg) -> Inc {
      const MwRec q = trs[t0 + i];
      reg = q.reg;
      return q.pad ? Inc{kBad, kBad} : Inc{q.e, q.o};
    };
    auto tile_desc = [&](int i, float &s2) -> long long {
      return serial((long long)c * kMwChunkTiles + t0 + i, s2);
    };
    return walk(kMwChunkTiles - t0, ss, cdf, r, tile_item, tile_desc);
  };
  // whole chunk c from memory values, serially (a skipped chunk reached anyway)
  auto chunk_serial = [&](int c, float &ss) -> long long {
    for (int t = 0; t < kMwChunkTiles; ++t) {
      const long long h = serial((long long)c * kMwChunkTiles + t, ss);
      if (h >= 0) return h;
    }
    return -1;
  };
  // apply run function F (region reg) from ss if valid and not hit; returns
  // false when the run has to be walked tile by tile instead
  auto apply_run = [&](uint32_t fe, uint32_t fo, int reg, float &ss) -> bool {
    const int rs = region_of(ss);
    if (!(reg == rs || reg == kAnyRegion)) return false;
    const uint32_t a0 = units_of(ss, rs);
    const uint32_t inc = inc_at(Inc{fe, fo}, a0);
    if (a0 + inc > kUnitsTop) return false;
    const float v = value_of(a0 + inc, rs);
    if (cdf && r <= v) return false;
    ss = v;
    return true;
  };

  for (int w0 = 1; w0 < a.NC && found < 0; w0 += kMwWin) {
    const int cnt = min(kMwWin, a.NC - w0);
    if (w0 > 1) {
      wave_sync();
      for (int c = lane; c < cnt; c += 64) cr[c] = crec[w0 + c];
      wave_sync();
    }
    auto chunk_item = [&](int i, int &reg) -> Inc {
      const MwChunk q = cr[i];
      reg = q.reg0;
      return (q.status == kChunkOk && q.brk < 0) ? Inc{q.e0, q.o0} : Inc{kBad, kBad};
    };
    auto chunk_desc = [&](int i, float &ss) -> long long {
      const MwChunk q = cr[i];
      const int c = w0 + i;
      if (q.status == kChunkSkipped) return chunk_serial(c, ss);
      if (q.status != kChunkOk || q.brk < 0) return tile_walk(c, 0, ss);
      const float s0 = ss;
      if (q.brk > 0 && !apply_run(q.e0, q.o0, q.reg0, ss)) {
        ss = s0;
        return tile_walk(c, 0, ss);
      }
      int t1 = q.brk;
      if (q.brk_serial) {
        const long long h = serial((long long)c * kMwChunkTiles + q.brk, ss);
        if (h >= 0) return h;
        ++t1;
      }
      if (t1 < kMwChunkTiles) {
        const float s1 = ss;
        if (!apply_run(q.e1, q.o1, q.reg1, ss)) {
          ss = s1;
          return tile_walk(c, t1, ss);
        }
      }
      return -1;
    };
    found = walk(cnt, s, cdf, r, chunk_item, chunk_desc);
  }
  if (lane == 0) {
    if (!cdf) {
      a.res[b].S = s;
      a.res[b].fallback = (s <= 1e-6f) ? 1 : 0;  // speculative.cpp:37
    } else {
      const int idx = (found < 0 || found >= a.V) ? a.V - 1 : (int)found;
      a.res[b].idx = idx;
      if (a.mode == CFA_MODE_CPP) finish_one(a, b, j, idx);
    }
  }
  // Python mode: past the end of the prefix sums, the last entry of
  // positive weight (the reference's C++ rule, V - 1, is kept in cpp mode).
  if (cdf && a.mode == CFA_MODE_PYTHON && found < 0) {
    const long long last = mw_last_positive(a, e);
    if (lane == 0) a.res[b].idx = (int)last;
  }
  return s;
}

// Everything after the first exact pass, kMwTailWGs work-groups ("parts")
// of kMwTailNT threads per job:
//   1. part 0's wave 0 (the walker) walks the sum pass (residual draws)
//      from chunk 1 on (the first pass walked chunk 0) and publishes S;
//   2. the walker writes the CDF pass's records of chunk 0 and walks it;
//      meanwhile the other waves of the job write the records of chunks
//      1 .. NC - 1 (chunk c to wave (c - 1) % 63 + 1 of the job's 64), from
//      entry values that one wave per part scans from the stored chunk sums;
//   3. the other parts report their shares done, and the walker walks the
//      rest of the CDF pass.
// A job's stages follow each other directly instead of in three launches
// (walk, records, walk), each of which waited for the slowest job of the
// previous one.
//
// S and the share counts cross work-groups (and XCDs) through agent-scope
// atomics on a.tsync, zeroed by the first kernel of the call: polled with
// relaxed loads, one release fence before each publication and one acquire
// fence after each wait (an acquire per poll would invalidate the cache on
// every poll).  The parts of a job take linear indices 8 apart, so that they
// share an XCD when work-groups go to the 8 XCDs round-robin.  Every wait is
// bounded, and none can cost correctness: a part that never sees S writes
// nothing, and a walker that does not see every share done writes the
// missing records itself -- the same values (the entry values come from the
// stored chunk sums, not from timing), so a late part's writes change
// nothing -- and then walks without the serial-tile cache, where a late part
// could still be filling a slot.
constexpr int kMwTailNT = 1024;
constexpr int kMwTailWaves = kMwTailNT / 64;
constexpr int kMwTailWGs = 4;
constexpr int kMwTailWorkers = kMwTailWGs * kMwTailWaves - 1;  // every wave but the walker
constexpr long kMwTailSpins = 1l << 15;  // s_sleep(2) polls: about 2 ms
constexpr unsigned long long kTsyncSet = 1ull << 63;  // a.tsync[2 b]: S is there

__device__ __forceinline__ unsigned long long ts_load(unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Job b and part of linear work-group index L: groups of 8 jobs take
// 8 * kMwTailWGs consecutive indices, the parts of one job 8 apart.
__device__ __forceinline__ void mw_tail_ids(int L, int &b, int &part) {
  const int grp = L / (8 * kMwTailWGs), w = L % (8 * kMwTailWGs);
  b = grp * 8 + (w % 8);
  part = w / 8;
}

__global__ __launch_bounds__(kMwTailNT) void mw_tail_kernel(Args a) {
  __shared__ MwWalkLds L;
  __shared__ float Es[kMwMaxNC];  // approximate chunk entry values (before the 1 / S)
  __shared__ float sS;
  __shared__ int sok;
  int b, part;
  mw_tail_ids(blockIdx.x, b, part);
  if (b >= a.B) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const MwJob j = a.jobs[b];
  if (!mw_active(j, kPassCdf)) {
    if (part == 0 && a.mode == CFA_MODE_CPP && threadIdx.x == 0) finish_one(a, b, j, -1);
    return;
  }
  const bool resid = j.kind == kResid;
  // a wave that does not walk scans the chunk sums of the CDF pass's row
  if (wave == 1) {
    const float *csum = (resid ? a.csum_x : a.csum_t) + (long long)b * a.NC;
    float carry = 0.0f;
    for (int base = 0; base < a.NC; base += 64) {
      const float v = (base + lane < a.NC) ? csum[base + lane] : 0.0f;
      const float incl = seq::wave_incl_scan_f32(v);
      if (base + lane < a.NC) Es[base + lane] = carry + (incl - v);
      carry += __shfl(incl, 63, 64);
    }
  }
  unsigned long long *ts = a.tsync + 2LL * b;
  MwRes r{0.0f, 0, -1, -1};
  if (resid) {
    if (part == 0) {
      if (wave == 0) {
        // chunk 0 was walked by the first pass (a.s0)
        const float S = mw_walk(a, b, kPassSum, j, mw_elem(a, b, j, kPassSum), L, true, true, a.s0[b]);
        if (lane == 0) {
          sS = S;
          __hip_atomic_store(ts, kTsyncSet | f2u(S), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    } else if (threadIdx.x == 0) {
      unsigned long long w = 0;
      for (long n = 0; n < kMwTailSpins; ++n) {
        w = ts_load(ts);
        if (w & kTsyncSet) break;
        __builtin_amdgcn_s_sleep(2);
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      sok = (w & kTsyncSet) ? 1 : 0;
      sS = u2f((uint32_t)w);
    }
    __syncthreads();
    if (part != 0 && !sok) return;  // the walker writes this part's share
    r.S = sS;
    r.fallback = (r.S <= 1e-6f) ? 1 : 0;  // speculative.cpp:37, as the walk stores it
  } else {
    __syncthreads();  // Es
  }
  const MwElem e = mw_elem_r(a, b, j, kPassCdf, r);
  // approximate entry value of chunk c on the CDF pass's scale (a residual
  // job whose sum fell to the fallback draws from t: t's own chunk sums)
  auto entry = [&](int c) __attribute__((always_inline)) -> float {
    if (resid && e.fn == 2) return mw_entry_prefix(a.csum_t + (long long)b * a.NC, c);
    return (e.fn == 1) ? Es[c] / e.S : Es[c];
  };
  // records of chunk c; a chunk surely past u gets a "skipped" record and no
  // loads.  Chunk 0 (never skipped: its entry value is 0) also goes to the
  // walker's LDS.
  auto records = [&](int c) __attribute__((always_inline)) {
    const float E0 = entry(c);
    if (mw_skip(kPassCdf, j, E0)) {
      mw_write_skipped(a, (long long)kPassCdf * a.B + b, c);
      return;
    }
    float x[kMwTile];
    mw_tile_values(a, e, (long long)c * kMwChunkTiles + lane, x);
    mw_records_chunk(a, b, c, kPassCdf, j, E0, x, c == 0 ? L.tr : nullptr, c == 0 ? L.xs : nullptr);
  };
  // worker gw = 16 part + wave (1 .. 16 kMwTailWGs - 1) writes chunks gw,
  // gw + kMwTailWorkers, ...; the walker (gw = 0) writes chunk 0 and walks it
  // at once, while the workers write the rest
  auto share_of = [&](int gw) __attribute__((always_inline)) {
    for (int c = gw; c < a.NC; c += kMwTailWorkers) records(c);
  };
  const int gw = part * kMwTailWaves + wave;
  float s0 = 0.0f;
  long long found0 = -1;
  if (gw == 0) {
    records(0);
    wave_sync();
    found0 = mw_walk_chunk0(L.xs, L.tr, true, j.u, s0);
  } else {
    share_of(gw);
  }
  if (part != 0) {
    // every wave's record stores complete, then one release for the part
    wait_vmcnt<0>();
    __syncthreads();
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __hip_atomic_fetch_add(ts + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long n = 0;
    for (long k = 0; k < kMwTailSpins; ++k) {
      n = ts_load(ts + 1);
      if (n >= (unsigned long long)(kMwTailWGs - 1)) break;
      __builtin_amdgcn_s_sleep(2);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    sok = (n >= (unsigned long long)(kMwTailWGs - 1)) ? 1 : 0;
  }
  __syncthreads();
  const bool all_in = sok != 0;
  if (!all_in) {
    for (int p = 1; p < kMwTailWGs; ++p) share_of(p * kMwTailWaves + wave);
    __syncthreads();
  }
  if (wave == 0) mw_walk(a, b, kPassCdf, j, e, L, all_in, true, s0, found0);
}

// ---------------------------------------------------------------------------
// python-mode bonus draw (top-p filter, renormalise, draw; speculative.py:
// 65-84): one work-group per sequence with the block-level exact replay.
// ---------------------------------------------------------------------------

constexpr int kSampleNT = 1024;

// Last index of positive weight (V - 1 if none): the block scans down from
// the end, NT elements per step (the rare fallback past the prefix sums).
template <int NT, class XF>
__device__ long long block_last_positive(const XF &xf, int V, int *slot) {
  for (long long base = ((long long)(V - 1) / NT) * NT; base >= 0; base -= NT) {
    __syncthreads();
    if (threadIdx.x == 0) *slot = -1;
    __syncthreads();
    const long long i = base + threadIdx.x;
    if (i < V && xf.eval(xf.load(i)) > 0.0f) atomicMax(slot, (int)i);
    __syncthreads();
    const int f = *slot;
    if (f >= 0) return f;
  }
  return V - 1;
}

__global__ __launch_bounds__(kSampleNT) void pybonus_kernel(Args a) {
  __shared__ seq::Shared<kSampleNT> sh;
  __shared__ double red[kSampleNT / 64];
  __shared__ int last;
  const int b = blockIdx.x, V = a.V;
  const MwJob j = a.jobs[b];
  // the bonus of a full acceptance, or the one after a rejection at K - 1
  if (j.kind != kPyBonus && !j.extra) return;
  const float u = (j.kind == kPyBonus) ? j.u : j.u2;
  const Dist t = make_dist(a, b, a.K);
  long long idx = -1;
  float vstar = (a.top_p < 1.0f) ? topp_threshold<kSampleNT>(t, V, a.top_p, red) : 0.0f;
  if (a.top_k > 0 && a.top_k < V) vstar = fmaxf(vstar, topk_threshold<kSampleNT>(t, V, a.top_k, red));
  const float S = seq::run<kSampleNT>(XKeep{t, vstar}, V, false, 0.0f, sh, nullptr);
  if (S > 0.0f) {
    const XKeepNorm xf{t, vstar, S};
    seq::run<kSampleNT>(xf, V, true, u, sh, &idx);
    if (idx < 0) idx = block_last_positive<kSampleNT>(xf, V, &last);
  } else {
    const XKeep xf{t, vstar};
    seq::run<kSampleNT>(xf, V, true, u, sh, &idx);
    if (idx < 0) idx = block_last_positive<kSampleNT>(xf, V, &last);
  }
  if (threadIdx.x == 0) {
    if (j.kind == kPyBonus)
      a.res[b].idx = (int)idx;
    else
      a.res[b].idx2 = (int)idx;
  }
}

// ---------------------------------------------------------------------------
// finish: per-sequence outputs.
// ---------------------------------------------------------------------------

// Outputs of sequence b; idx is the drawn token (ignored without a draw).
// idx2: the python-mode bonus that follows a resample (j.extra).
__device__ __forceinline__ void finish_one(const Args &a, int b, const MwJob &j, int idx,
                                           int idx2) {
  const int K = a.K;
  const int n = j.n, eos_acc = j.eos_acc;
  int fin = (j.kind == kNone) ? -1 : idx;
  int32_t *ot = a.out_tokens + (long long)b * (K + 1);
  for (int q = 0; q <= K; ++q) {
    int v = -1;
    if (q < n) v = a.tokens[(long long)b * K + q];
    if (q == n && !eos_acc) v = fin;
    if (q == n + 1 && j.extra) v = idx2;
    ot[q] = v;
  }
  if (eos_acc) fin = a.eos;
  if (j.extra) fin = idx2;  // the last token emitted
  a.out_accept_len[b] = n;
  a.out_final[b] = fin;
  a.out_eos[b] = (a.mode == CFA_MODE_CPP) ? ((eos_acc || fin == a.eos) ? 1 : 0) : 0;
  a.out_num_emitted[b] = eos_acc ? n : n + 1 + (j.extra ? 1 : 0);
}

// Python mode (cpp mode finishes each sequence at the end of its last walk).
__global__ __launch_bounds__(64) void finish_kernel(Args a) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b >= a.B) return;
  const MwJob j = a.jobs[b];
  const MwRes r = a.res[b];
  finish_one(a, b, j, r.idx, r.idx2);
}

// Optional: write the probabilities the verification used.
__global__ __launch_bounds__(256) void probs_out_kernel(Args a, float *out_t, float *out_d) {
  const int r = blockIdx.y;
  const int b = r / a.rpb, j = r % a.rpb;
  float *dst = (j <= a.K) ? out_t + ((long long)b * (a.K + 1) + j) * a.V
                          : out_d + ((long long)b * a.K + (j - a.K - 1)) * a.V;
  if ((j <= a.K && !out_t) || (j > a.K && !out_d)) return;
  const Dist d = make_dist_u(a, b, j);
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < a.V; i += (long long)gridDim.x * 256)
    dst[i] = d(i);
}

// ---------------------------------------------------------------------------
// Greedy top-k of raw rows (k <= kTopKMax): the k largest values, largest
// first, equal values by lower index (sampling.h:107-135 for k = 1).
// Pass 1: grid (splits, rows), each work-group the top-k of its slice;
// pass 2: one thread per row merges the splits' lists.
// ---------------------------------------------------------------------------

constexpr int kTopKMax = 8;

__device__ __forceinline__ bool tk_better(float v, int i, float w, int j) {
  return v > w || (v == w && i < j);
}

template <int K>
__device__ __forceinline__ void tk_insert(float (&v)[K], int (&ix)[K], float x, int i) {
  if (!tk_better(x, i, v[K - 1], ix[K - 1])) return;
#pragma unroll
  for (int s = K - 1; s >= 0; --s) {
    const bool shift = (s > 0) && tk_better(x, i, v[s - 1], ix[s - 1]);
    if (shift) {
      v[s] = v[s - 1];
      ix[s] = ix[s - 1];
    } else {
      v[s] = x;
      ix[s] = i;
      break;
    }
  }
}

struct TopKArgs {
  const float *x;
  long long stride;
  int R, V, k, splits;
  long long per_split;
  float2 *part;  // [R, splits, k] (value, index as bits)
  int32_t *out;  // [R, k]
};

template <int NT>
__global__ __launch_bounds__(NT) void topk_partial_kernel(TopKArgs a) {
  __shared__ float sv[NT * kTopKMax];
  __shared__ int si[NT * kTopKMax];
  const int r = blockIdx.y, sp = blockIdx.x;
  const float *row = a.x + (long long)r * a.stride;
  const long long e0 = (long long)sp * a.per_split;
  const long long e1 = min((long long)a.V, e0 + a.per_split);
  float v[kTopKMax];
  int ix[kTopKMax];
#pragma unroll
  for (int q = 0; q < kTopKMax; ++q) {
    v[q] = -INFINITY;
    ix[q] = 0x7fffffff;
  }
  for (long long i = e0 + threadIdx.x; i < e1; i += NT) {
    const float x = __builtin_nontemporal_load(row + i);
    if (x == x) tk_insert<kTopKMax>(v, ix, x, (int)i);  // NaN never ranks
  }
  // tree merge of the threads' lists through LDS
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < kTopKMax; ++q) {
    sv[t * kTopKMax + q] = v[q];
    si[t * kTopKMax + q] = ix[q];
  }
  for (int half = NT / 2; half >= 1; half >>= 1) {
    __syncthreads();
    if (t < half) {
      const int o = (t + half) * kTopKMax;
      for (int q = 0; q < a.k; ++q) tk_insert<kTopKMax>(v, ix, sv[o + q], si[o + q]);
#pragma unroll
      for (int q = 0; q < kTopKMax; ++q) {
        sv[t * kTopKMax + q] = v[q];
        si[t * kTopKMax + q] = ix[q];
      }
    }
  }
  __syncthreads();
  if (t < a.k) {
    float2 *dst = a.part + ((long long)r * a.splits + sp) * a.k;
    dst[t] = make_float2(sv[t], __int_as_float(si[t]));
  }
}

__global__ __launch_bounds__(64) void topk_merge_kernel(TopKArgs a) {
  const int r = blockIdx.x * 64 + threadIdx.x;
  if (r >= a.R) return;
  float v[kTopKMax];
  int ix[kTopKMax];
#pragma unroll
  for (int q = 0; q < kTopKMax; ++q) {
    v[q] = -INFINITY;
    ix[q] = 0x7fffffff;
  }
  const float2 *src = a.part + (long long)r * a.splits * a.k;
  for (int e = 0; e < a.splits * a.k; ++e) tk_insert<kTopKMax>(v, ix, src[e].x, __float_as_int(src[e].y));
  for (int q = 0; q < a.k; ++q)
    a.out[(long long)r * a.k + q] = (ix[q] == 0x7fffffff) ? (q == 0 ? 0 : -1) : ix[q];
}

}  // namespace chain
}  // namespace cfa

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
using namespace cfa;
using namespace cfa::chain;

static size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

// Slices per row of the stats / argmax passes: slices of at most 16384
// vector units (256 KiB of fp32 at 16-byte loads; 128 KiB slices measured
// 1% slower at C2, 64 KiB 9%), and for few rows enough slices for about
// 1024 work-groups (slices of at least 256 units).  A function of the shape
// only, so every pass over a row combines the same partials in the same
// order.
// Work-groups per CU of the balanced tail pass (1 and 2 measured slower;
// busy work-groups need other waves beside them on their CU to keep enough
// loads in flight).
constexpr int kTailPerCU = 3;
static int stats_slices(long long R, long long Vw) {
  const long long by_len = (Vw + 16383) / 16384;
  const long long by_rows = std::min<long long>((1024 + R - 1) / R, std::max<long long>(1, Vw / 256));
  return (int)std::min<long long>(256, std::max<long long>(1, std::max(by_len, by_rows)));
}
// Head positions of the two-pass statistics (cpp rules, logits): with the
// ~0.7 per-position acceptance of typical draft models, 3 minimises the rows
// the two passes read together.
constexpr int kHeadPositions = 3;

// Workspace layout (each region 256-byte aligned).
struct WsLayout {
  size_t part, apart, rawtok, dec, ufin, jobs, res, csum_x, csum_t, crec, trec, badcnt, bad, x0, flags,
      tsync, s0, total;
};

static WsLayout ws_layout(int B, int K, int V, int mode) {
  const int rpb = (mode == CFA_MODE_GREEDY) ? K + 1 : 2 * K + 1;
  const size_t R = (size_t)B * rpb;
  const size_t G = R * (size_t)stats_slices((long long)R, V);  // the largest slice count (scalar loads)
  const size_t NC = (size_t)((V + kMwChunk - 1) / kMwChunk);
  const bool mw = mode != CFA_MODE_GREEDY;
  WsLayout L{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align_up(bytes);
    return at;
  };
  L.part = take(G * sizeof(float2));
  L.apart = take(G * sizeof(float2));
  L.rawtok = take(R * sizeof(float));
  L.dec = take((size_t)B * sizeof(int4));
  L.ufin = take((size_t)B * sizeof(float));
  L.jobs = take((size_t)B * sizeof(MwJob));
  L.res = take((size_t)B * sizeof(MwRes));
  L.csum_x = take(mw ? (size_t)B * NC * sizeof(float) : 0);
  L.csum_t = take(mw ? (size_t)B * NC * sizeof(float) : 0);
  L.crec = take(mw ? 2 * (size_t)B * NC * sizeof(MwChunk) : 0);
  L.trec = take(mw ? 2 * (size_t)B * NC * kMwChunkTiles * sizeof(MwRec) : 0);
  L.badcnt = take(2 * (size_t)B * sizeof(int));
  L.bad = take(mw ? 2 * (size_t)B * kMwMaxBad * sizeof(MwBad) : 0);
  L.x0 = take(mw ? 2 * (size_t)B * kMwChunk * sizeof(float) : 0);
  L.flags = take(mw ? (size_t)B * NC * sizeof(unsigned long long) : 0);
  L.tsync = take(2 * (size_t)B * sizeof(unsigned long long));
  L.s0 = take((size_t)B * sizeof(float));
  L.total = o;
  return L;
}

extern "C" size_t cfa_chain_verify_workspace_size(int B, int K, int V, int input_kind, int mode) {
  (void)input_kind;
  if (B <= 0 || K < 0 || V <= 0) return 0;
  return ws_layout(B, K, V, mode).total;
}

static int run_pipeline(Args &a, bool vec, void *workspace, hipStream_t st, float *out_target_probs,
                        float *out_draft_probs);

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
  if ((long long)V > (long long)kMwMaxNC * kMwChunk) return fail_arg("V must be at most 4194304");
  if (B > 65535) return fail_arg("B must be at most 65535");
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
  a.ustride = (mode == CFA_MODE_PYTHON) ? K + 2 : K + 1;
  a.B = B;
  a.K = K;
  a.V = V;
  a.draws = 1;
  a.rpb = (mode == CFA_MODE_GREEDY) ? K + 1 : 2 * K + 1;
  a.logits = input_kind == CFA_INPUT_LOGITS;
  a.c = a.logits ? (float)(1.4426950408889634 / (double)temperature) : 1.0f;
  a.mode = mode;
  a.eos = eos_token_id;
  // top_p <= 0 keeps only the most probable token, as speculative.py:72-76
  // does for any top_p below the largest probability; NaN filters nothing
  a.top_p = (top_p != top_p) ? 1.0f : fmaxf(top_p, 0.0f);
  a.top_k = 0;
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
  return run_pipeline(a, vec, workspace, (hipStream_t)stream, out_target_probs, out_draft_probs);
}

// Partition, workspace carve-up and launches shared by chain verification
// and the sampler.  a.B jobs read a.B / a.draws row groups of a.rpb rows.
static int run_pipeline(Args &a, bool vec, void *workspace, hipStream_t st, float *out_target_probs,
                        float *out_draft_probs) {
  using namespace cfa::abi;
  const int B = a.B, K = a.K, V = a.V, mode = a.mode;
  const int W = vec ? 4 : 1;
  a.Vw = V / W;
  const int R = (B / a.draws) * a.rpb;
  a.R = R;
  a.S = stats_slices(R, a.Vw);
  // cpp rules with logits: statistics in two passes, the second only for the
  // sequences that accepted every head position (not when the caller asks
  // for every row's probabilities)
  const bool two_pass = mode == CFA_MODE_CPP && a.logits && a.draws == 1 && K > kHeadPositions &&
                        !out_target_probs && !out_draft_probs;
  a.P = two_pass ? kHeadPositions : K;

  a.vec = vec ? 1 : 0;
  a.NC = (V + kMwChunk - 1) / kMwChunk;
  const WsLayout L = ws_layout(B, K, V, mode);
  char *ws = (char *)workspace;
  a.part = (float2 *)(ws + L.part);
  a.apart = (float2 *)(ws + L.apart);
  a.rawtok = (float *)(ws + L.rawtok);
  a.dec = (int4 *)(ws + L.dec);
  a.ufin = (float *)(ws + L.ufin);
  a.jobs = (MwJob *)(ws + L.jobs);
  a.res = (MwRes *)(ws + L.res);
  a.csum_x = (float *)(ws + L.csum_x);
  a.csum_t = (float *)(ws + L.csum_t);
  a.crec = (MwChunk *)(ws + L.crec);
  a.trec = (MwRec *)(ws + L.trec);
  a.badcnt = (int *)(ws + L.badcnt);
  a.bad = (MwBad *)(ws + L.bad);
  a.x0 = (float *)(ws + L.x0);
  a.flags = (unsigned long long *)(ws + L.flags);
  a.tsync = (unsigned long long *)(ws + L.tsync);
  a.s0 = (float *)(ws + L.s0);
  // the first statistics pass zeroes the look-back words, cache counters and
  // tail synchronisation words; without one (probabilities input) a small
  // kernel does
  a.mw_reset = (mode != CFA_MODE_GREEDY && a.logits) ? 1 : 0;

  if (mode != CFA_MODE_GREEDY && !a.logits) {
    const long long n = std::max<long long>((long long)B * a.NC, 2LL * B);
    const int grid = (int)std::min<long long>((n + 255) / 256, 1024);
    CFA_LAUNCH("chain_mw_reset", mw_reset_kernel, dim3(grid), dim3(256), 0, st, a);
  }
  if (a.logits) {
    const int groups = R / a.rpb;
    auto stats = [&](int set, int entries) -> int {
      const dim3 grid((unsigned)entries, (unsigned)a.S);
      const char *name = set == kRowsHead ? "chain_stats_head"
                         : set == kRowsTail ? "chain_stats_tail" : "chain_stats";
      if (vec)
        CFA_LAUNCH(name, (stats_kernel<kStatsNT, 4>), grid, dim3(kStatsNT), 0, st, a, set);
      else
        CFA_LAUNCH(name, (stats_kernel<kStatsNT, 1>), grid, dim3(kStatsNT), 0, st, a, set);
      return CFA_OK;
    };
    int rc;
    if (two_pass) {
      if ((rc = stats(kRowsHead, groups * 2 * a.P)) != CFA_OK) return rc;
      if (vec && groups <= kTailMaxGroups) {
        const long long items = (long long)groups * (2 * (K - a.P) + 1) * a.S;
        const int grid = (int)std::min<long long>(items, (long long)kTailPerCU * device_cu_count());
        CFA_LAUNCH("chain_stats_tail", stats_tail_kernel<kStatsNT>, dim3(grid), dim3(kStatsNT), 0, st, a);
      } else if ((rc = stats(kRowsTail, groups * (2 * (K - a.P) + 1))) != CFA_OK) {
        return rc;
      }
    } else if ((rc = stats(kRowsAll, R)) != CFA_OK) {
      return rc;
    }
  }
  if (mode == CFA_MODE_GREEDY)
    CFA_LAUNCH("chain_argmax", (argmax_kernel<256>), dim3((unsigned)R, (unsigned)a.S), dim3(256), 0,
               st, a);
  // cpp rules: the mw sums kernel takes each sequence's decision itself
  const int fused_decide = mode == CFA_MODE_CPP ? 1 : 0;
  if (!fused_decide) CFA_LAUNCH("chain_decide", decide_kernel, dim3(B), dim3(64), 0, st, a);
  if (mode != CFA_MODE_GREEDY) {
    const dim3 cg1((a.NC + kMwChunksPerWG - 1) / kMwChunksPerWG, B);   // two chunks per wave
    const unsigned tail_wgs = (unsigned)(((B + 7) / 8) * 8 * kMwTailWGs);
    if (mode == CFA_MODE_PYTHON) CFA_LAUNCH("chain_plan", plan_kernel, dim3(1), dim3(256), 0, st, a);
    CFA_LAUNCH("chain_mw_first", mw_first_kernel, cg1, dim3(kMwNT), 0, st, a, fused_decide);
    CFA_LAUNCH("chain_mw_tail", mw_tail_kernel, dim3(tail_wgs), dim3(kMwTailNT), 0, st, a);
    if (mode == CFA_MODE_PYTHON)
      CFA_LAUNCH("chain_pybonus", pybonus_kernel, dim3(B), dim3(kSampleNT), 0, st, a);
    if (mode == CFA_MODE_PYTHON)
      CFA_LAUNCH("chain_finish", finish_kernel, dim3((B + 63) / 64), dim3(64), 0, st, a);
  }
  if (out_target_probs || out_draft_probs) {
    const int gx = std::min(64, (V + 255) / 256);
    CFA_LAUNCH("chain_probs_out", probs_out_kernel, dim3(gx, R), dim3(256), 0, st, a,
               out_target_probs, out_draft_probs);
  }
  return CFA_OK;
}

// ---------------------------------------------------------------------------
// Sampler: plain decode and draft-tree expansion.
// ---------------------------------------------------------------------------

static int topk_splits(int R, int V) {
  const int want = std::max(1, (1024 + R - 1) / R);
  return std::max(1, std::min(want, V / 2048));
}

static int sample_chain_mode(int mode) {
  return mode == CFA_SAMPLE_FILTERED ? CFA_MODE_PYTHON : CFA_MODE_CPP;
}

extern "C" size_t cfa_sample_workspace_size(int R, int V, int draws, int mode) {
  if (R <= 0 || V <= 0 || draws <= 0) return 0;
  if (mode == CFA_SAMPLE_GREEDY)
    return align_up((size_t)R * topk_splits(R, V) * draws * sizeof(float2));
  const size_t B = (size_t)R * draws;
  return ws_layout((int)B, 0, V, sample_chain_mode(mode)).total + 3 * align_up(B * sizeof(int32_t));
}

extern "C" int cfa_sample(const float *rows, int64_t row_stride, int input_kind, int R, int V,
                          int draws, float temperature, int top_k, float top_p, int mode,
                          const float *uniforms, int32_t *out_tokens, float *out_probs,
                          void *workspace, size_t workspace_bytes, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (R <= 0 || V <= 0 || draws <= 0) return fail_arg("R, V and draws must be positive");
  if ((long long)V > (long long)kMwMaxNC * kMwChunk) return fail_arg("V must be at most 4194304");
  if ((long long)R * draws > 65535) return fail_arg("R * draws must be at most 65535");
  if (mode != CFA_SAMPLE_MULTINOMIAL && mode != CFA_SAMPLE_FILTERED && mode != CFA_SAMPLE_GREEDY)
    return fail_arg("mode must be CFA_SAMPLE_MULTINOMIAL, CFA_SAMPLE_FILTERED or CFA_SAMPLE_GREEDY");
  if (input_kind != CFA_INPUT_PROBS && input_kind != CFA_INPUT_LOGITS)
    return fail_arg("input_kind must be CFA_INPUT_PROBS or CFA_INPUT_LOGITS");
  if (!rows || !out_tokens) return fail_arg("null pointer");
  if (row_stride < V) return fail_arg("row_stride must be at least V");
  const size_t need = cfa_sample_workspace_size(R, V, draws, mode);
  if (!workspace || workspace_bytes < need) return fail_arg("workspace too small (see cfa_sample_workspace_size)");
  hipStream_t st = (hipStream_t)stream;

  if (mode == CFA_SAMPLE_GREEDY) {
    if (draws > kTopKMax) return fail_arg("greedy sampling returns at most 8 tokens per row");
    if (draws > V) return fail_arg("draws must not exceed V");
    if (out_probs) return fail_arg("out_probs is not produced in greedy mode");
    TopKArgs t{};
    t.x = rows;
    t.stride = row_stride;
    t.R = R;
    t.V = V;
    t.k = draws;
    t.splits = topk_splits(R, V);
    t.per_split = (V + t.splits - 1) / t.splits;
    t.part = (float2 *)workspace;
    t.out = out_tokens;
    CFA_LAUNCH("sample_topk", (topk_partial_kernel<256>), dim3(t.splits, R), dim3(256), 0, st, t);
    CFA_LAUNCH("sample_topk_merge", topk_merge_kernel, dim3((R + 63) / 64), dim3(64), 0, st, t);
    return CFA_OK;
  }
  if (!uniforms) return fail_arg("null uniforms");
  if (input_kind == CFA_INPUT_LOGITS && !(temperature > 0.0f)) return fail_arg("temperature must be > 0");
  if (mode == CFA_SAMPLE_FILTERED && !(top_p > 0.0f && top_p <= 1.0f))
    return fail_arg("top_p must be in (0, 1]");

  const int B = R * draws;
  const int chain_mode = sample_chain_mode(mode);
  Args a{};
  a.tgt = rows;
  a.t_sb = row_stride;
  a.t_sk = V;
  a.drf = nullptr;
  a.tokens = nullptr;
  a.U = uniforms;
  a.ustride = 1;  // one uniform per draw
  a.B = B;
  a.K = 0;
  a.V = V;
  a.draws = draws;
  a.rpb = 1;
  a.logits = input_kind == CFA_INPUT_LOGITS;
  a.c = a.logits ? (float)(1.4426950408889634 / (double)temperature) : 1.0f;
  a.mode = chain_mode;
  a.eos = -1;
  a.top_p = (mode == CFA_SAMPLE_FILTERED) ? top_p : 1.0f;
  a.top_k = (mode == CFA_SAMPLE_FILTERED) ? top_k : 0;
  const WsLayout L = ws_layout(B, 0, V, chain_mode);
  char *tail = (char *)workspace + L.total;
  const size_t ib = align_up((size_t)B * sizeof(int32_t));
  a.out_tokens = out_tokens;
  a.out_final = (int32_t *)tail;
  a.out_accept_len = (int32_t *)(tail + ib);
  a.out_num_emitted = (int32_t *)(tail + 2 * ib);
  a.out_eos = a.out_accept_len;  // written after out_accept_len, never read
  const bool vec = (V % 4 == 0) && (row_stride % 4 == 0) && (((uintptr_t)rows & 15) == 0);
  return run_pipeline(a, vec, workspace, st, out_probs, nullptr);
}

// ---------------------------------------------------------------------------
// Allocation-free chain verification.  Its workspace is a file-scope device
// array, so a caller that cannot allocate (HIP graph capture, a serving loop
// that forbids allocation) passes only inputs and outputs.  Every GPU the
// library runs on holds its own copy of the array until the process ends;
// calls on one GPU share it, so calls that overlap on one GPU (different
// streams, or host threads) race.  Nothing in it has to start at zero: every
// region the pipeline reads is written earlier in the same call.
// ---------------------------------------------------------------------------

constexpr size_t kScratchBytes = size_t(32) << 20;  // 32 MiB: B = 64, K = 8, V = 128256 needs 18.7
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device
}  // namespace

// The current device's address of `scratch`, looked up once per device (the
// host-side name of the array is not a device address).
static int scratch_ptr(void **out) {
  using namespace cfa::abi;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail_arg("device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail_code(CFA_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CFA_OK;
}

extern "C" int cfa_chain_verify_noalloc(const float *target, int64_t t_stride_b,
                                        int64_t t_stride_k, const float *draft,
                                        int64_t d_stride_b, int64_t d_stride_k, int input_kind,
                                        const int32_t *draft_tokens, const float *uniforms, int B,
                                        int K, int V, float temperature, float top_p, int mode,
                                        int32_t eos_token_id, int32_t *out_accept_len,
                                        int32_t *out_tokens, int32_t *out_num_emitted,
                                        int32_t *out_final, int32_t *out_eos,
                                        float *out_target_probs, float *out_draft_probs,
                                        void *stream) {
  using namespace cfa::abi;
  clear_error();
  const size_t need = cfa_chain_verify_workspace_size(B, K, V, input_kind, mode);
  if (need > kScratchBytes)
    return fail_arg("cfa_chain_verify_noalloc: this shape needs more than the 32 MiB static "
                    "scratch (see cfa_chain_verify_workspace_size); use cfa_chain_verify with "
                    "a workspace");
  void *ws = nullptr;
  if (const int rc = scratch_ptr(&ws)) return rc;
  return cfa_chain_verify(target, t_stride_b, t_stride_k, draft, d_stride_b, d_stride_k,
                          input_kind, draft_tokens, uniforms, B, K, V, temperature, top_p, mode,
                          eos_token_id, out_accept_len, out_tokens, out_num_emitted, out_final,
                          out_eos, out_target_probs, out_draft_probs, ws, kScratchBytes, stream);
}
