// llama_ops.hip -- fused element-wise layers around the verify step's
// attention: residual add + RMSNorm, rotary embedding fused with the KV-cache
// write, and SiLU-gated product.  All bf16 in HBM with fp32 arithmetic; each
// replaces a chain of PyTorch kernels with one pass over the activations.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include "abi_internal.hpp"
#include "silu.hpp"

namespace cfa {
namespace ops {

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// ---------------------------------------------------------------------------
// h <- bf16(h + delta) (when delta is given); out <- bf16(h * rsqrt(mean(h^2)
// + eps) * w).  One work-group per row; thread t takes the 4-element vectors
// (8 bytes of bf16, 16 of fp32) t, t + 256, ... in that order, so that every
// wave access is contiguous, and sums its squares in that order before the
// block reduction (both kernels below: the same bits).
// ---------------------------------------------------------------------------
constexpr int kNormNT = 256;

// x (4 bf16) += the 4 values of d, each rounded to bf16 first; squares into ss
__device__ __forceinline__ void norm_fold(uint2 &x, float d0, float d1, float d2, float d3,
                                          float &ss) {
  const float a0 = bf2f(x.x & 0xffff) + d0, a1 = bf2f(x.x >> 16) + d1;
  const float a2 = bf2f(x.y & 0xffff) + d2, a3 = bf2f(x.y >> 16) + d3;
  x.x = (uint32_t)f2bf(a0) | ((uint32_t)f2bf(a1) << 16);
  x.y = (uint32_t)f2bf(a2) | ((uint32_t)f2bf(a3) << 16);
}
__device__ __forceinline__ void norm_sq(const uint2 &x, float &ss) {
  const float a0 = bf2f(x.x & 0xffff), a1 = bf2f(x.x >> 16);
  const float a2 = bf2f(x.y & 0xffff), a3 = bf2f(x.y >> 16);
  ss += a0 * a0 + a1 * a1;
  ss += a2 * a2 + a3 * a3;
}
__device__ __forceinline__ uint2 norm_scale(const uint2 &x, const uint2 &g, float inv) {
  uint2 o;
  o.x = (uint32_t)f2bf(bf2f(x.x & 0xffff) * inv * bf2f(g.x & 0xffff)) |
        ((uint32_t)f2bf(bf2f(x.x >> 16) * inv * bf2f(g.x >> 16)) << 16);
  o.y = (uint32_t)f2bf(bf2f(x.y & 0xffff) * inv * bf2f(g.y & 0xffff)) |
        ((uint32_t)f2bf(bf2f(x.y >> 16) * inv * bf2f(g.y >> 16)) << 16);
  return o;
}
// rsqrt(mean + eps) of the row from every thread's ss (fixed order)
__device__ __forceinline__ float norm_inv(float ss, int d, float eps) {
  __shared__ float red[kNormNT / 64];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormNT / 64; ++i) tot += red[i];
  return rsqrtf(tot / (float)d + eps);
}

__global__ __launch_bounds__(kNormNT) void rmsnorm_kernel(uint16_t *h, const uint16_t *delta,
                                                          const uint16_t *w, uint16_t *out, int d,
                                                          float eps) {
  const long long row = blockIdx.x;
  uint2 *hr = reinterpret_cast<uint2 *>(h + row * d);
  const uint2 *dr = delta ? reinterpret_cast<const uint2 *>(delta + row * d) : nullptr;
  uint2 *orow = reinterpret_cast<uint2 *>(out + row * d);
  const uint2 *wr = reinterpret_cast<const uint2 *>(w);
  const int nvec = d / 4;
  float ss = 0.0f;
  for (int v = threadIdx.x; v < nvec; v += kNormNT) {
    uint2 x = hr[v];
    if (dr) {
      const uint2 y = dr[v];
      norm_fold(x, bf2f(y.x & 0xffff), bf2f(y.x >> 16), bf2f(y.y & 0xffff), bf2f(y.y >> 16), ss);
      hr[v] = x;
    }
    norm_sq(x, ss);
  }
  const float inv = norm_inv(ss, d, eps);
  for (int v = threadIdx.x; v < nvec; v += kNormNT) orow[v] = norm_scale(hr[v], wr[v], inv);
}

// Sum, in slab order, of S fp32 slabs (4 consecutive values at p, p + slab,
// ...): S > 0 a compile-time count, every load issued before the first add
// (the sum is then one memory latency, not S); S == 0 the runtime count n.
template <int S>
__device__ __forceinline__ float4 slab_sum4(const float *p, long long slab, int n) {
  if constexpr (S > 0) {
    float4 v[S];
#pragma unroll
    for (int k = 0; k < S; ++k) v[k] = *reinterpret_cast<const float4 *>(p + k * slab);
    float4 acc = v[0];
#pragma unroll
    for (int k = 1; k < S; ++k) {
      acc.x += v[k].x;
      acc.y += v[k].y;
      acc.z += v[k].z;
      acc.w += v[k].w;
    }
    return acc;
  } else {
    float4 acc = *reinterpret_cast<const float4 *>(p);
    for (int k = 1; k < n; ++k) {
      const float4 t = *reinterpret_cast<const float4 *>(p + k * slab);
      acc.x += t.x;
      acc.y += t.y;
      acc.z += t.z;
      acc.w += t.w;
    }
    return acc;
  }
}

__device__ __forceinline__ void norm_fold_part(uint2 &x, const float4 &p, float &ss) {
  norm_fold(x, bf2f(f2bf(p.x)), bf2f(f2bf(p.y)), bf2f(f2bf(p.z)), bf2f(f2bf(p.w)), ss);
}

// rmsnorm_kernel with delta = bf16 of the sum of the split-K partials
// part[s][M][d] (slab order) -- what the W4A16 GEMM's reduce writes, so the
// partials need no separate pass; the same bits.  For d <= 4 * 4 * kNormNT
// (4 vectors per thread) every load -- the partials, h and the weights -- is
// issued before the first use and h stays in registers for the output.
template <int S>
__global__ __launch_bounds__(kNormNT) void rmsnorm_part_kernel(uint16_t *h, const float *part,
                                                               const uint16_t *w, uint16_t *out,
                                                               int d, float eps, long long slab,
                                                               int splits) {
  constexpr int kV = 4;
  const long long row = blockIdx.x;
  uint2 *hr = reinterpret_cast<uint2 *>(h + row * d);
  const float *pr = part + row * d;
  uint2 *orow = reinterpret_cast<uint2 *>(out + row * d);
  const uint2 *wr = reinterpret_cast<const uint2 *>(w);
  const int nvec = d / 4;
  float ss = 0.0f;
  if (nvec <= kV * kNormNT) {
    float4 p[kV];
    uint2 x[kV], g[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) {  // clamped: every load issued and in bounds
      const int c = min((int)threadIdx.x + k * kNormNT, nvec - 1);
      p[k] = slab_sum4<S>(pr + 4 * c, slab, splits);
      x[k] = hr[c];
      g[k] = wr[c];
    }
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int v = threadIdx.x + k * kNormNT;
      if (v < nvec) {
        norm_fold_part(x[k], p[k], ss);
        hr[v] = x[k];
        norm_sq(x[k], ss);
      }
    }
    const float inv = norm_inv(ss, d, eps);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int v = threadIdx.x + k * kNormNT;
      if (v < nvec) orow[v] = norm_scale(x[k], g[k], inv);
    }
    return;
  }
  for (int v = threadIdx.x; v < nvec; v += kNormNT) {
    uint2 x = hr[v];
    norm_fold_part(x, slab_sum4<S>(pr + 4 * v, slab, splits), ss);
    hr[v] = x;
    norm_sq(x, ss);
  }
  const float inv = norm_inv(ss, d, eps);
  for (int v = threadIdx.x; v < nvec; v += kNormNT) orow[v] = norm_scale(hr[v], wr[v], inv);
}

// ---------------------------------------------------------------------------
// Rotary embedding (rotate-half pairs (i, i + D/2), angle pos * theta^(-2i/D))
// of the q and k heads of a fused [M, Hq + 2 Hkv, D] projection, fused with
// the write of k and v into the KV cache:
//   q_out [M, Hq, D] (contiguous);
//   paged cache (kind 0): token m = b * n + j goes to slot base[b] + j of
//     pool[block][layer][kv_head][slot_in_block][D], block =
//     block_tables[b][slot / bs] (an unmapped page, -1 or past max_blocks,
//     is skipped);
//   strided cache (kind 1): k to kc + b*k_sb + h*k_sh + slot*k_ss + e*k_se,
//     v to vc + b*v_sb + h*v_sh + slot*v_ss + e (slot = slots[m]).
// One thread per (token, head, rotation pair).
// ---------------------------------------------------------------------------
struct RopeArgs {
  const uint16_t *qkv;
  const int32_t *pos;   // [M]
  uint16_t *q_out;
  uint16_t *kc, *vc;
  int M, n, Hq, Hkv, D;
  float log2_theta;
  int kind;
  // paged
  const int32_t *block_tables;
  int max_blocks, bs, layer;
  const int32_t *base;
  long long blk_stride, layer_stride, head_stride;  // elements
  // strided
  const int32_t *slots;  // [M]
  long long k_sb, k_sh, k_ss, k_se, v_sb, v_sh, v_ss;
  // qkv given as `splits` fp32 slabs part[s][M][H * D] (split-K partials of
  // the W4A16 GEMM) instead: element = bf16 of their sum in slab order
  const float *part;
  int splits;
  long long slab;
};

// bf16 bits of elements idx .. idx + P - 1 of the fused projection (P = 4:
// one 8-byte bf16 load, or one 16-byte load per fp32 slab)
template <int P, int S>
__device__ __forceinline__ void qkv_load(const RopeArgs &a, long long idx, uint16_t (&v)[P]) {
  if constexpr (P == 4) {
    if (a.part) {
      const float4 s = slab_sum4<S>(a.part + idx, a.slab, a.splits);
      v[0] = f2bf(s.x);
      v[1] = f2bf(s.y);
      v[2] = f2bf(s.z);
      v[3] = f2bf(s.w);
    } else {
      const uint2 w = *reinterpret_cast<const uint2 *>(a.qkv + idx);
      v[0] = (uint16_t)w.x;
      v[1] = (uint16_t)(w.x >> 16);
      v[2] = (uint16_t)w.y;
      v[3] = (uint16_t)(w.y >> 16);
    }
  } else {
#pragma unroll
    for (int k = 0; k < P; ++k) {
      if (!a.part) {
        v[k] = a.qkv[idx + k];
        continue;
      }
      float x = a.part[idx + k];
      for (int sp = 1; sp < a.splits; ++sp) x += a.part[sp * a.slab + idx + k];
      v[k] = f2bf(x);
    }
  }
}

// P contiguous bf16 values to dst (P = 4: one 8-byte store)
template <int P>
__device__ __forceinline__ void store_p(uint16_t *dst, const uint16_t (&v)[P]) {
  if constexpr (P == 4) {
    *reinterpret_cast<uint2 *>(dst) =
        make_uint2((uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16));
  } else {
#pragma unroll
    for (int k = 0; k < P; ++k) dst[k] = v[k];
  }
}

// One thread per (token, head, P consecutive rotation pairs), or per P
// consecutive v elements; P = 4 when D / 2 % 4 == 0 and the buffers are
// 16-byte aligned, else 1.  Every element is computed the same way for both P.
template <int P, int S>
__global__ __launch_bounds__(256) void rope_kv_kernel(RopeArgs a) {
  const int half = a.D / 2, hp = half / P, dp = a.D / P;
  const int H = a.Hq + 2 * a.Hkv;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long total = (long long)a.M * (a.Hq + a.Hkv) * hp;
  const long long tv = (long long)a.M * a.Hkv * dp;
  if (t >= total + tv) return;
  if (t >= total) {  // v copy
    const long long r = t - total;
    const int e0 = (int)(r % dp) * P;
    const int h = (int)((r / dp) % a.Hkv);
    const int m = (int)(r / ((long long)dp * a.Hkv));
    uint16_t val[P];
    qkv_load<P, S>(a, ((long long)m * H + a.Hq + a.Hkv + h) * a.D + e0, val);
    const int b = m / a.n, j = m % a.n;
    if (a.kind == 0) {
      const int slot = a.base[b] + j;
      if (slot / a.bs >= a.max_blocks) return;
      const long long blk = a.block_tables[(long long)b * a.max_blocks + slot / a.bs];
      if (blk < 0) return;  // unmapped page: never written
      store_p<P>(a.vc + blk * a.blk_stride + a.layer * a.layer_stride + h * a.head_stride +
                     (long long)(slot % a.bs) * a.D + e0,
                 val);
    } else {
      const long long slot = a.slots[m];
      store_p<P>(a.vc + b * a.v_sb + h * a.v_sh + slot * a.v_ss + e0, val);
    }
    return;
  }
  const int i0 = (int)(t % hp) * P;
  const int hh = (int)((t / hp) % (a.Hq + a.Hkv));
  const int m = (int)(t / ((long long)hp * (a.Hq + a.Hkv)));
  const long long src = ((long long)m * H + hh) * a.D;
  uint16_t lo[P], hi[P], y0[P], y1[P];
  qkv_load<P, S>(a, src + i0, lo);
  qkv_load<P, S>(a, src + i0 + half, hi);
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const int i = i0 + k;
    const float x0 = bf2f(lo[k]), x1 = bf2f(hi[k]);
    const float inv_freq = exp2f(-(float)(2 * i) / (float)a.D * a.log2_theta);
    const float ang = (float)a.pos[m] * inv_freq;
    float sn, cs;
    sincosf(ang, &sn, &cs);
    y0[k] = f2bf(x0 * cs - x1 * sn);
    y1[k] = f2bf(x1 * cs + x0 * sn);
  }
  if (hh < a.Hq) {
    uint16_t *dst = a.q_out + ((long long)m * a.Hq + hh) * a.D;
    store_p<P>(dst + i0, y0);
    store_p<P>(dst + i0 + half, y1);
    return;
  }
  const int h = hh - a.Hq;
  const int b = m / a.n, j = m % a.n;
  if (a.kind == 0) {
    const int slot = a.base[b] + j;
    if (slot / a.bs >= a.max_blocks) return;
    const long long blk = a.block_tables[(long long)b * a.max_blocks + slot / a.bs];
    if (blk < 0) return;
    uint16_t *dst = a.kc + blk * a.blk_stride + a.layer * a.layer_stride + h * a.head_stride +
                    (long long)(slot % a.bs) * a.D;
    store_p<P>(dst + i0, y0);
    store_p<P>(dst + i0 + half, y1);
  } else {
    const long long slot = a.slots[m];
    uint16_t *dst = a.kc + b * a.k_sb + h * a.k_sh + slot * a.k_ss;
#pragma unroll
    for (int k = 0; k < P; ++k) {
      dst[(long long)(i0 + k) * a.k_se] = y0[k];
      dst[(long long)(i0 + k + half) * a.k_se] = y1[k];
    }
  }
}

static int launch_rope(const RopeArgs &a, void *stream) {
  // four pairs per thread where every access of four elements is aligned
  // (the strided cache's v rows: v_ss a multiple of 4 as well)
  const bool aligned =
      (((uintptr_t)a.qkv | (uintptr_t)a.part | (uintptr_t)a.q_out | (uintptr_t)a.kc |
        (uintptr_t)a.vc) & 15) == 0 &&
      (a.kind == 0 || (a.v_sb % 4 == 0 && a.v_sh % 4 == 0 && a.v_ss % 4 == 0));
  const int P = (a.D % 8 == 0 && aligned) ? 4 : 1;
  const long long total =
      (long long)a.M * (a.Hq + a.Hkv) * (a.D / 2 / P) + (long long)a.M * a.Hkv * (a.D / P);
  const dim3 grid((unsigned)((total + 255) / 256));
  // the 8B target's QKV projection splits K five ways: its partial sums get
  // a compile-time slab count (every load in flight at once)
  if (P == 4 && a.part && a.splits == 5)
    CFA_LAUNCH("rope_kv", (rope_kv_kernel<4, 5>), grid, dim3(256), 0, (hipStream_t)stream, a);
  else if (P == 4)
    CFA_LAUNCH("rope_kv", (rope_kv_kernel<4, 0>), grid, dim3(256), 0, (hipStream_t)stream, a);
  else
    CFA_LAUNCH("rope_kv", (rope_kv_kernel<1, 0>), grid, dim3(256), 0, (hipStream_t)stream, a);
  return CFA_OK;
}

// out[m, f] = bf16(bf16(silu(g)) * u) for gu [M, 2F] = [g | u] (the rounding
// of silu(g) * u in two bf16 PyTorch ops; silu_gate).
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *gu, uint16_t *out, int M,
                                                       int F) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)M * F) return;
  const long long m = t / F, f = t % F;
  out[t] = silu_gate(bf2f(gu[m * 2 * F + f]), bf2f(gu[m * 2 * F + F + f]));
}

// The same, eight features per thread with 16-byte loads and stores
// (F % 8 == 0, 16-byte aligned gu and out).
__global__ __launch_bounds__(256) void silu_mul8_kernel(const uint16_t *gu, uint16_t *out, int M,
                                                        int F) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const int F8 = F / 8;
  if (t >= (long long)M * F8) return;
  const long long m = t / F8, f = (t % F8) * 8;
  const uint4 gv = *reinterpret_cast<const uint4 *>(gu + m * 2 * F + f);
  const uint4 uv = *reinterpret_cast<const uint4 *>(gu + m * 2 * F + F + f);
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t ow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ow[j] = silu_gate2(silu_lo(gw[j]), silu_lo(uw[j]), silu_hi(gw[j]), silu_hi(uw[j]));
  }
  *reinterpret_cast<uint4 *>(out + m * F + f) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

}  // namespace ops
}  // namespace cfa

using namespace cfa::ops;

extern "C" int cfa_rmsnorm(void *h, const void *delta, const void *weight, void *out, int M, int d,
                           float eps, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (M <= 0 || d <= 0 || d % 8 != 0) return fail_arg("M > 0 and d a positive multiple of 8");
  if (!h || !weight || !out) return fail_arg("null pointer");
  if ((((uintptr_t)h | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)delta) & 15) != 0)
    return fail_arg("rows must be 16-byte aligned");
  CFA_LAUNCH("rmsnorm", rmsnorm_kernel, dim3(M), dim3(kNormNT), 0, (hipStream_t)stream,
             (uint16_t *)h, (const uint16_t *)delta, (const uint16_t *)weight, (uint16_t *)out, d,
             eps);
  return CFA_OK;
}

extern "C" int cfa_rmsnorm_partials(void *h, const float *part, int splits, const void *weight,
                                    void *out, int M, int d, float eps, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (M <= 0 || d <= 0 || d % 8 != 0) return fail_arg("M > 0 and d a positive multiple of 8");
  if (splits <= 0) return fail_arg("splits must be positive");
  if (!h || !part || !weight || !out) return fail_arg("null pointer");
  if ((((uintptr_t)h | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)part) & 15) != 0)
    return fail_arg("rows must be 16-byte aligned");
  const long long slab = (long long)M * d;
#define CFA_NORM_PART(S)                                                                     \
  CFA_LAUNCH("rmsnorm", rmsnorm_part_kernel<S>, dim3(M), dim3(kNormNT), 0, (hipStream_t)stream, \
             (uint16_t *)h, part, (const uint16_t *)weight, (uint16_t *)out, d, eps, slab, splits)
  switch (splits) {
    case 1: CFA_NORM_PART(1); break;
    case 2: CFA_NORM_PART(2); break;
    case 4: CFA_NORM_PART(4); break;
    case 5: CFA_NORM_PART(5); break;
    case 8: CFA_NORM_PART(8); break;
    default: CFA_NORM_PART(0); break;
  }
#undef CFA_NORM_PART
  return CFA_OK;
}

static int rope_paged(const void *qkv, const float *part, int splits, const int32_t *positions,
                      int B, int n, int Hq, int Hkv, int D, float theta, void *q_out,
                      void *k_pool, void *v_pool, int layer, int num_layers, int block_size,
                      const int32_t *block_tables, int max_blocks, const int32_t *base_lens,
                      void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || D % 2) return fail_arg("bad shape");
  if (layer < 0 || layer >= num_layers || block_size <= 0) return fail_arg("bad layer or block size");
  if ((!qkv && !part) || !positions || !q_out || !k_pool || !v_pool || !block_tables || !base_lens)
    return fail_arg("null pointer");
  if (part && splits <= 0) return fail_arg("splits must be positive");
  RopeArgs a{};
  a.qkv = (const uint16_t *)qkv;
  a.part = part;
  a.splits = splits;
  a.slab = (long long)B * n * (Hq + 2 * Hkv) * D;
  a.pos = positions;
  a.q_out = (uint16_t *)q_out;
  a.kc = (uint16_t *)k_pool;
  a.vc = (uint16_t *)v_pool;
  a.M = B * n;
  a.n = n;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = D;
  a.log2_theta = log2f(theta);
  a.kind = 0;
  a.block_tables = block_tables;
  a.max_blocks = max_blocks;
  a.bs = block_size;
  a.layer = layer;
  a.base = base_lens;
  a.head_stride = (long long)block_size * D;
  a.layer_stride = (long long)Hkv * a.head_stride;
  a.blk_stride = (long long)num_layers * a.layer_stride;
  return launch_rope(a, stream);
}

extern "C" int cfa_rope_kv_paged(const void *qkv, const int32_t *positions, int B, int n, int Hq,
                                 int Hkv, int D, float theta, void *q_out, void *k_pool,
                                 void *v_pool, int layer, int num_layers, int block_size,
                                 const int32_t *block_tables, int max_blocks,
                                 const int32_t *base_lens, void *stream) {
  return rope_paged(qkv, nullptr, 0, positions, B, n, Hq, Hkv, D, theta, q_out, k_pool, v_pool,
                    layer, num_layers, block_size, block_tables, max_blocks, base_lens, stream);
}

extern "C" int cfa_rope_kv_paged_partials(const float *part, int splits, const int32_t *positions,
                                          int B, int n, int Hq, int Hkv, int D, float theta,
                                          void *q_out, void *k_pool, void *v_pool, int layer,
                                          int num_layers, int block_size,
                                          const int32_t *block_tables, int max_blocks,
                                          const int32_t *base_lens, void *stream) {
  if (!part) {
    cfa::abi::clear_error();
    return cfa::abi::fail_arg("null pointer");
  }
  return rope_paged(nullptr, part, splits, positions, B, n, Hq, Hkv, D, theta, q_out, k_pool,
                    v_pool, layer, num_layers, block_size, block_tables, max_blocks, base_lens,
                    stream);
}

extern "C" int cfa_rope_kv_strided(const void *qkv, const int32_t *positions, int B, int n, int Hq,
                                   int Hkv, int D, float theta, void *q_out, void *k_cache,
                                   const int64_t *k_strides, void *v_cache,
                                   const int64_t *v_strides, const int32_t *slots, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || D % 2) return fail_arg("bad shape");
  if (!qkv || !positions || !q_out || !k_cache || !v_cache || !slots || !k_strides || !v_strides)
    return fail_arg("null pointer");
  if (v_strides[3] != 1) return fail_arg("v rows must be contiguous");
  RopeArgs a{};
  a.qkv = (const uint16_t *)qkv;
  a.pos = positions;
  a.q_out = (uint16_t *)q_out;
  a.kc = (uint16_t *)k_cache;
  a.vc = (uint16_t *)v_cache;
  a.M = B * n;
  a.n = n;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = D;
  a.log2_theta = log2f(theta);
  a.kind = 1;
  a.slots = slots;
  a.k_sb = k_strides[0];
  a.k_sh = k_strides[1];
  a.k_ss = k_strides[2];
  a.k_se = k_strides[3];
  a.v_sb = v_strides[0];
  a.v_sh = v_strides[1];
  a.v_ss = v_strides[2];
  return launch_rope(a, stream);
}

extern "C" int cfa_silu_mul(const void *gu, void *out, int M, int F, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (M <= 0 || F <= 0) return fail_arg("bad shape");
  if (!gu || !out) return fail_arg("null pointer");
  const long long total = (long long)M * F;
  if (F % 8 == 0 && (((uintptr_t)gu | (uintptr_t)out) & 15) == 0) {
    const long long items = total / 8;
    CFA_LAUNCH("silu_mul", silu_mul8_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
               (hipStream_t)stream, (const uint16_t *)gu, (uint16_t *)out, M, F);
  } else {
    CFA_LAUNCH("silu_mul", silu_mul_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
               (hipStream_t)stream, (const uint16_t *)gu, (uint16_t *)out, M, F);
  }
  return CFA_OK;
}
