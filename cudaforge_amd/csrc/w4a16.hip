// w4a16.hip -- INT4 weight dequantisation (W4A16, group-wise scales).
//
// Weight format of the reference (csrc/include/cudaforge/kernels/
// dequantize.cuh:12-25, tests/unit/test_int4_dequant.py:6-15): B_quant
// [K / 8, N] 32-bit words, nibble (k % 8) of word (k / 8, n) at bits
// 4 * (k % 8), unsigned 0..15; scales [K / group, N] fp16; optional zero
// points [K / group, N] fp16.  Dequantised value (int4_gemm_dequant.cu:20-31):
//   fp16:  w = (fp16(nibble) - z) * s in fp16 arithmetic (each step rounded),
//          and without zero points w = fp16(nibble * s), the value
//          int4_dequant_triton.py:74-78 produces;
//   bf16:  w = bf16((nibble - z) * s) with the product formed in fp32.
// Each thread takes four adjacent packed words (one 16-byte read) and writes
// 8 rows of four outputs (8-byte stores); a one-word-per-thread kernel covers
// unaligned or N % 4 != 0 shapes.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include "abi_internal.hpp"
#include "lds_dma.hpp"

namespace cfa {
namespace w4 {

struct Args {
  const uint32_t *q;   // [K/8, N]
  const __half *s;     // [K/g, N]
  const __half *z;     // [K/g, N] or null
  void *out;           // [K, N]
  int K, N, group;
  int bf16;
};

__device__ __forceinline__ uint16_t to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);  // round to nearest even
}

__device__ __forceinline__ void dequant_word(const Args &a, uint32_t w, __half sh, __half zh,
                                             long long row0, int n) {
  if (a.bf16) {
    uint16_t *o = reinterpret_cast<uint16_t *>(a.out);
    const float sf = __half2float(sh), zf = __half2float(zh);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float nib = (float)((w >> (4 * i)) & 15u);
      o[(row0 + i) * a.N + n] = to_bf16_bits((nib - zf) * sf);
    }
  } else {
    __half *o = reinterpret_cast<__half *>(a.out);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const __half nib = __float2half((float)((w >> (4 * i)) & 15u));
      o[(row0 + i) * a.N + n] = __hmul(__hsub(nib, zh), sh);
    }
  }
}

// One thread per packed word.
__global__ __launch_bounds__(256) void dequant_kernel(Args a) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long words = (long long)(a.K / 8) * a.N;
  if (idx >= words) return;
  const int kb = (int)(idx / a.N), n = (int)(idx % a.N);
  const int g = (kb * 8) / a.group;
  const __half sh = a.s[(long long)g * a.N + n];
  const __half zh = a.z ? a.z[(long long)g * a.N + n] : __float2half(0.0f);
  dequant_word(a, a.q[idx], sh, zh, (long long)kb * 8, n);
}

// Four adjacent columns per thread (N % 4 == 0, 16-byte aligned words):
// one 16-byte read of words, 8-byte writes of each output row.
__global__ __launch_bounds__(256) void dequant4_kernel(Args a) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const int N4 = a.N / 4;
  const long long quads = (long long)(a.K / 8) * N4;
  if (idx >= quads) return;
  const int kb = (int)(idx / N4), n = (int)(idx % N4) * 4;
  const int g = (kb * 8) / a.group;
  const uint4 w = *reinterpret_cast<const uint4 *>(a.q + (long long)kb * a.N + n);
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  __half sh[4], zh[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    sh[c] = a.s[(long long)g * a.N + n + c];
    zh[c] = a.z ? a.z[(long long)g * a.N + n + c] : __float2half(0.0f);
  }
  uint16_t r[8][4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (a.bf16) {
      const float sf = __half2float(sh[c]), zf = __half2float(zh[c]);
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i][c] = to_bf16_bits(((float)((ws[c] >> (4 * i)) & 15u) - zf) * sf);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const __half nib = __float2half((float)((ws[c] >> (4 * i)) & 15u));
        r[i][c] = __half_as_ushort(__hmul(__hsub(nib, zh[c]), sh[c]));
      }
    }
  }
  uint16_t *o = reinterpret_cast<uint16_t *>(a.out);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint2 v;
    v.x = (uint32_t)r[i][0] | ((uint32_t)r[i][1] << 16);
    v.y = (uint32_t)r[i][2] | ((uint32_t)r[i][3] << 16);
    *reinterpret_cast<uint2 *>(o + ((long long)kb * 8 + i) * a.N + n) = v;
  }
}

// Transposed output out [N, K] (K contiguous, the layout hipBLASLt
// multiplies fastest as the second operand).  A work-group covers 64 packed
// rows x CT columns (CT = 64 for large matrices, 16 where 64 would leave
// fewer than 1024 work-groups).  Load phase: the words (16 bytes per thread when
// VEC) go into an LDS block padded to CT + 1 words a row, with the
// block's scale (and zero-point) rows when there are at most kDqtGroups of
// them.  Store phase, LDS only: lane l of wave w takes packed row kb0 + l
// of columns n0 + (CT/4) w .. n0 + (CT/4)(w + 1) - 1 (the odd row pitch keeps those column
// reads free of bank conflicts), and each output store of the wave writes
// 64 consecutive 16-byte chunks of one row of out (1 KiB contiguous).
// Consecutive work-groups take consecutive k-blocks of the same rows of
// out, so the writes in flight fill whole rows.
constexpr int kDqtGroups = 8;

template <int CT, bool VEC>
__global__ __launch_bounds__(256) void dequant_t_kernel(Args a) {
  constexpr int kDqtCols = CT, kDqtPitch = CT + 1;
  __shared__ uint32_t blk[64 * kDqtPitch];
  __shared__ __half sblk[kDqtGroups * kDqtCols], zblk[kDqtGroups * kDqtCols];  // [group - g0][column]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kb0 = blockIdx.x * 64, n0 = blockIdx.y * kDqtCols;
  const int KB = a.K / 8;
  const int g0 = (kb0 * 8) / a.group;
  const int g1 = (min(kb0 + 64, KB) * 8 - 1) / a.group;  // last group of the block
  if (VEC) {
#pragma unroll
    for (int j = 0; j < CT / 16; ++j) {
      const int i = tid + 256 * j;
      const int r = i / (CT / 4), c = 4 * (i % (CT / 4));
      const int kb = kb0 + r, n = n0 + c;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (kb < KB && n < a.N) v = *reinterpret_cast<const uint4 *>(a.q + (long long)kb * a.N + n);
      uint32_t *d = blk + r * kDqtPitch + c;
      d[0] = v.x;
      d[1] = v.y;
      d[2] = v.z;
      d[3] = v.w;
    }
  } else {
    for (int i = tid; i < 64 * kDqtCols; i += 256) {
      const int r = i / kDqtCols, c = i % kDqtCols;
      const int kb = kb0 + r, n = n0 + c;
      blk[r * kDqtPitch + c] = (kb < KB && n < a.N) ? a.q[(long long)kb * a.N + n] : 0u;
    }
  }
  const bool staged = g1 - g0 < kDqtGroups;
  for (int i = tid; staged && i < (g1 - g0 + 1) * kDqtCols; i += 256) {
    const int gi = i / kDqtCols, n = n0 + i % kDqtCols;
    const long long src = (long long)(g0 + gi) * a.N + n;
    sblk[i] = n < a.N ? a.s[src] : __float2half(0.0f);
    zblk[i] = (a.z && n < a.N) ? a.z[src] : __float2half(0.0f);
  }
  __syncthreads();
  const int kb = kb0 + lane;
  if (kb >= KB) return;
  const int gi = (kb * 8) / a.group - g0;
  uint16_t *o = reinterpret_cast<uint16_t *>(a.out);
#pragma unroll
  for (int c = 0; c < kDqtCols / 4; ++c) {
    const int col = (kDqtCols / 4) * wave + c, n = n0 + col;
    if (n >= a.N) break;
    const uint32_t w = blk[lane * kDqtPitch + col];
    __half sh, zh;
    if (staged) {
      sh = sblk[gi * kDqtCols + col];
      zh = zblk[gi * kDqtCols + col];
    } else {
      sh = a.s[(long long)(g0 + gi) * a.N + n];
      zh = a.z ? a.z[(long long)(g0 + gi) * a.N + n] : __float2half(0.0f);
    }
    uint16_t r[8];
    if (a.bf16) {
      const float sf = __half2float(sh), zf = __half2float(zh);
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = to_bf16_bits(((float)((w >> (4 * i)) & 15u) - zf) * sf);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const __half nib = __float2half((float)((w >> (4 * i)) & 15u));
        r[i] = __half_as_ushort(__hmul(__hsub(nib, zh), sh));
      }
    }
    uint4 v;
    v.x = (uint32_t)r[0] | ((uint32_t)r[1] << 16);
    v.y = (uint32_t)r[2] | ((uint32_t)r[3] << 16);
    v.z = (uint32_t)r[4] | ((uint32_t)r[5] << 16);
    v.w = (uint32_t)r[6] | ((uint32_t)r[7] << 16);
    *reinterpret_cast<uint4 *>(o + (long long)n * a.K + (long long)kb * 8) = v;
  }
}

}  // namespace w4
}  // namespace cfa

extern "C" int cfa_w4a16_dequant_t(const uint32_t *b_quant, const void *scales, const void *zeros,
                                   int K, int N, int group_size, int out_bf16, void *out,
                                   void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (K <= 0 || N <= 0 || group_size <= 0) return fail_arg("K, N and group_size must be positive");
  if (K % 8 != 0) return fail_arg("K must be a multiple of 8");
  if (group_size % 8 != 0 || K % group_size != 0)
    return fail_arg("group_size must be a multiple of 8 that divides K");
  if (!b_quant || !scales || !out) return fail_arg("null pointer");
  if ((uintptr_t)out & 15) return fail_arg("out must be 16-byte aligned");
  cfa::w4::Args a{};
  a.q = b_quant;
  a.s = (const __half *)scales;
  a.z = (const __half *)zeros;
  a.out = out;
  a.K = K;
  a.N = N;
  a.group = group_size;
  a.bf16 = out_bf16 ? 1 : 0;
  const unsigned kblocks = (unsigned)((K / 8 + 63) / 64);
  const bool wide = (long long)kblocks * ((N + 63) / 64) >= 1024;
  const int ct = wide ? 64 : 16;
  const dim3 grid(kblocks, (unsigned)((N + ct - 1) / ct));
  const bool vec = N % 4 == 0 && ((uintptr_t)b_quant & 15) == 0;
  hipStream_t st = (hipStream_t)stream;
  if (wide && vec)
    CFA_LAUNCH("w4a16_dequant_t", (cfa::w4::dequant_t_kernel<64, true>), grid, dim3(256), 0, st, a);
  else if (wide)
    CFA_LAUNCH("w4a16_dequant_t", (cfa::w4::dequant_t_kernel<64, false>), grid, dim3(256), 0, st, a);
  else if (vec)
    CFA_LAUNCH("w4a16_dequant_t", (cfa::w4::dequant_t_kernel<16, true>), grid, dim3(256), 0, st, a);
  else
    CFA_LAUNCH("w4a16_dequant_t", (cfa::w4::dequant_t_kernel<16, false>), grid, dim3(256), 0, st, a);
  return CFA_OK;
}

extern "C" int cfa_w4a16_dequant(const uint32_t *b_quant, const void *scales, const void *zeros,
                                 int K, int N, int group_size, int out_bf16, void *out,
                                 void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (K <= 0 || N <= 0 || group_size <= 0) return fail_arg("K, N and group_size must be positive");
  if (K % 8 != 0) return fail_arg("K must be a multiple of 8");
  if (group_size % 8 != 0 || K % group_size != 0)
    return fail_arg("group_size must be a multiple of 8 that divides K");
  if (!b_quant || !scales || !out) return fail_arg("null pointer");
  cfa::w4::Args a{};
  a.q = b_quant;
  a.s = (const __half *)scales;
  a.z = (const __half *)zeros;
  a.out = out;
  a.K = K;
  a.N = N;
  a.group = group_size;
  a.bf16 = out_bf16 ? 1 : 0;
  const bool vec = (N % 4 == 0) && (((uintptr_t)b_quant & 15) == 0) && (((uintptr_t)out & 7) == 0);
  const long long items = (long long)(K / 8) * (vec ? N / 4 : N);
  const long long blocks = (items + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail_arg("matrix too large");
  if (vec)
    CFA_LAUNCH("w4a16_dequant", cfa::w4::dequant4_kernel, dim3((unsigned)blocks), dim3(256), 0,
               (hipStream_t)stream, a);
  else
    CFA_LAUNCH("w4a16_dequant", cfa::w4::dequant_kernel, dim3((unsigned)blocks), dim3(256), 0,
               (hipStream_t)stream, a);
  return CFA_OK;
}

// ---------------------------------------------------------------------------
// Fused W4A16 GEMM: C [M, N] = A [M, K] x dequant(B_quant) for bf16 or fp16
// activations, fp32 accumulation on v_mfma_f32_16x16x32_{bf16,f16}.
//
// Work-group tile BM x 256 (BM = 64 or 32), four waves of BM x 64, K in steps
// of 64.  Each step's A tile (16-byte chunks XOR-swizzled by row, for
// conflict-free MFMA operand reads), packed weights and scale row move by
// direct HBM -> LDS transfers into a 4-stage ring, three steps ahead, with
// one barrier per step.  Lane l of a wave reads, per 32-k half step, the four
// adjacent words of columns n0 + 4 (l % 16) + j (j = 0..3) at packed row
// k0/8 + l/16 -- one 16-byte LDS read -- and word j, dequantised in
// registers, is exactly the lane's 8-element B fragment of the wave's n-tile
// j, whose column c is global column n0 + 4c + j.  Dequantisation is the bf16 / fp16
// formula of dequant_kernel, so the result equals dequantise-then-GEMM up to
// the order of the fp32 accumulation.
// ---------------------------------------------------------------------------
namespace cfa {
namespace w4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct GArgs {
  const uint16_t *A;   // [M, K]
  const uint32_t *q;   // [K/8, N]
  const __half *s;     // [K/g, N]
  uint16_t *C;         // [M, N]
  int M, N, K, group;
  int mtiles, ntiles;
};

constexpr int kGBN = 256, kGBK = 64;

template <bool F16>
__device__ __forceinline__ void dequant_frag(uint32_t w, float s, uint32_t (&out)[4]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float f0 = (float)((w >> (8 * p)) & 15u) * s;
    const float f1 = (float)((w >> (8 * p + 4)) & 15u) * s;
    uint32_t lo, hi;
    if (F16) {
      lo = __half_as_ushort(__float2half(f0));
      hi = __half_as_ushort(__float2half(f1));
    } else {
      lo = __builtin_bit_cast(uint16_t, (__bf16)f0);
      hi = __builtin_bit_cast(uint16_t, (__bf16)f1);
    }
    out[p] = lo | (hi << 16);
  }
}

template <int BM, bool F16>
__global__ __launch_bounds__(256, 2) void w4gemm_kernel(GArgs a) {
  constexpr int MT = BM / 16;                   // 16-row MFMA tiles per wave
  constexpr int kS = 4, kP = 3;                 // ring stages, iterations in flight
  constexpr int ABYTES = BM * kGBK * 2;         // A tile (128-byte rows)
  constexpr int BBYTES = (kGBK / 8) * kGBN * 4; // 8 packed rows of 256 words
  constexpr int SBYTES = kGBN * 2;              // one scale row
  constexpr int STAGE = ABYTES + BBYTES + SBYTES;
  constexpr int AX = ABYTES / 1024 / 4;         // A transfers per wave
  constexpr int LPI = AX + 2 + 1;               // transfers per wave per iteration
  __shared__ __align__(16) uint8_t ring[kS * STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Work-groups go to the 8 XCDs round-robin by linear index; the m-tiles of
  // one n-tile take indices 8 apart, so they share an XCD and its L2, which
  // then serves their common weight columns.
  const int L = blockIdx.x;
  const int ntile = (L % 8) + 8 * (L / (8 * a.mtiles));
  const int mti = (L / 8) % a.mtiles;
  if (ntile >= a.ntiles) return;  // padding of the last group of 8 n-tiles
  const int m0 = mti * BM;
  const int nbase = ntile * kGBN;
  const int iters = a.K / kGBK;

  // this lane's sources of the per-iteration transfers (k0 added per issue)
  const uint16_t *asrc[AX];
#pragma unroll
  for (int j = 0; j < AX; ++j) {
    const int x = wave * AX + j;                  // 1 KiB transfer: A rows 8x .. 8x + 7
    const int row = 8 * x + (lane >> 3);
    const int c = (lane & 7) ^ (row & 7);         // chunk landing at position lane % 8
    asrc[j] = a.A + (long long)min(m0 + row, a.M - 1) * a.K + 8 * c;
  }
  const uint32_t *bsrc = a.q + (long long)(2 * wave) * a.N + nbase + 4 * lane;
  const __half *ssrc = a.s + nbase + 64 * wave + 8 * (lane & 7);

  auto issue = [&](int u) {
    uint8_t *st = ring + (u % kS) * STAGE;
    const int k0 = u * kGBK;
#pragma unroll
    for (int j = 0; j < AX; ++j)
      dma16(asrc[j] + k0, (CFA_LDS void *)(st + 1024 * (wave * AX + j)));
#pragma unroll
    for (int j = 0; j < 2; ++j)
      dma16(bsrc + (long long)(k0 / 8 + j) * a.N,
            (CFA_LDS void *)(st + ABYTES + 1024 * (2 * wave + j)));
    if (lane < 8)
      dma16(ssrc + (long long)(k0 / a.group) * a.N, (CFA_LDS void *)(st + ABYTES + BBYTES + 128 * wave));
  };

  f32x4 acc[MT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int u = 0; u < min(kP, iters); ++u) issue(u);
  for (int it = 0; it < iters; ++it) {
    const int later = min(kP - 1, iters - 1 - it);  // iterations issued after this one
    if (later >= 2) wait_vmcnt<2 * LPI>();
    else if (later == 1) wait_vmcnt<LPI>();
    else wait_vmcnt<0>();
    block_barrier();  // every wave's part of stage `it` has landed
    // the stage refilled here was last read in iteration it - 1
    if (it + kP < iters) issue(it + kP);
    const uint8_t *st = ring + (it % kS) * STAGE;
    const uint2 sv = *reinterpret_cast<const uint2 *>(st + ABYTES + BBYTES + (64 * wave + 4 * (lane & 15)) * 2);
    float sc[4];
    sc[0] = __half2float(__ushort_as_half((uint16_t)(sv.x & 0xffff)));
    sc[1] = __half2float(__ushort_as_half((uint16_t)(sv.x >> 16)));
    sc[2] = __half2float(__ushort_as_half((uint16_t)(sv.y & 0xffff)));
    sc[3] = __half2float(__ushort_as_half((uint16_t)(sv.y >> 16)));
    const uint4 *Ab = reinterpret_cast<const uint4 *>(st);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint4 bw = *reinterpret_cast<const uint4 *>(
          st + ABYTES + (4 * s + (lane >> 4)) * 1024 + (64 * wave + 4 * (lane & 15)) * 4);
      const uint32_t wj[4] = {bw.x, bw.y, bw.z, bw.w};
      uint32_t bf[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) dequant_frag<F16>(wj[j], sc[j], bf[j]);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int row = 16 * i + (lane & 15);
        const int kc = s * 4 + (lane >> 4);
        const uint4 av = Ab[row * 8 + (kc ^ (row & 7))];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 bv = make_uint4(bf[j][0], bf[j][1], bf[j][2], bf[j][3]);
          if (F16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // C[row][n0 + 4c + j] = acc[i][j][e], row = m0 + 16 i + 4 (lane / 16) + e
  const int bcol = nbase + 64 * wave + 4 * (lane & 15);
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + 16 * i + 4 * (lane >> 4) + e;
      if (row >= a.M) continue;
      uint16_t v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (F16)
          v[j] = __half_as_ushort(__float2half(acc[i][j][e]));
        else
          v[j] = __builtin_bit_cast(uint16_t, (__bf16)acc[i][j][e]);
      }
      uint2 w;
      w.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
      w.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
      *reinterpret_cast<uint2 *>(a.C + (long long)row * a.N + bcol) = w;
    }
}

// ---------------------------------------------------------------------------
// Fused W4A16 GEMM with cooperative dequantisation (bf16 activations), the
// form for many rows (the verify step's M = 504).  Work-group tile 128 x BN
// (BN = 128, or 64 where 128 would leave CUs idle), K in steps of 64, four
// waves of 64 x BN/2.  Each step's A tile (128 rows x 64 k, 16-byte chunks
// XOR-swizzled by row), packed words (8 rows x BN) and scale row move by
// direct HBM -> LDS transfers into a 3-stage ring two steps ahead.  The 256
// threads then dequantise the step's 64 x BN weights once, into an LDS tile
// laid out [n][k] (one 16-byte write per packed word, chunks swizzled by
// column), from which every wave reads its B operands with 16-byte reads.
// Dequantisation is bf16(nibble * scale) formed in fp32, as
// cfa_w4a16_dequant, so the result equals dequantise-then-GEMM up to the
// order of the fp32 accumulation.  Two work-groups share a CU, so one's
// dequantisation overlaps the other's MFMAs.
// ---------------------------------------------------------------------------
constexpr int kW2BM = 128, kW2BK = 64;

template <int BN, int ST>
struct W2Cfg {
  static constexpr int kABytes = kW2BM * kW2BK * 2;     // 16 KiB
  static constexpr int kQBytes = (kW2BK / 8) * BN * 4;  // 8 packed rows
  static constexpr int kSBytes = BN * 2;                // one scale row
  static constexpr int kStage = kABytes + kQBytes + kSBytes;
  static constexpr int kStages = ST;
  static constexpr int kBBytes = BN * kW2BK * 2;        // dequantised tile [n][k]
  static constexpr int kLPI = 4 + 1 + 1;                // transfers per wave per stage
  static constexpr int kNB = BN / 32;                   // 16-column blocks per wave
  static constexpr int kWords = BN / 32;                // packed words per thread per stage
  static_assert(ST > 3 || kStages * kStage + kBBytes <= 80 * 1024, "two work-groups per CU");
  static_assert(kStages * kStage + kBBytes <= 160 * 1024, "LDS");
};

template <int N>
__device__ __forceinline__ void w2_wait() {  // vmcnt(N) lgkmcnt(0)
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | (((N >> 4) & 3) << 14));
}
// vmcnt(n * LPI) lgkmcnt(0) for a run-time 0 <= n <= N
template <int LPI, int N>
__device__ __forceinline__ void w2_wait_stages(int n) {
  if constexpr (N == 0) {
    w2_wait<0>();
  } else {
    if (n >= N) w2_wait<N * LPI>();
    else w2_wait_stages<LPI, N - 1>(n);
  }
}

template <int BN, int ST>
__global__ __launch_bounds__(256, 2) void w4g2_kernel(GArgs a) {
  using Cf = W2Cfg<BN, ST>;
  constexpr int kS = Cf::kStages, kP = kS - 1, LPI = Cf::kLPI, NB = Cf::kNB, NW = Cf::kWords;
  __shared__ __align__(16) uint8_t ring[kS * Cf::kStage];
  __shared__ __align__(16) uint8_t btile[Cf::kBBytes];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  // the m-tiles of one n-tile take linear indices 8 apart: one XCD, whose
  // L2 then serves their common packed weights
  const int L = blockIdx.x;
  const int ntile = (L % 8) + 8 * (L / (8 * a.mtiles));
  const int mti = (L / 8) % a.mtiles;
  if (ntile >= a.ntiles) return;
  const int m0 = mti * kW2BM, n0 = ntile * BN;
  const int iters = a.K / kW2BK;

  // transfer sources (the step's k offset is added per issue)
  const uint16_t *asrc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * (4 * wave + j) + (lane >> 3);  // 1 KiB = 8 rows of A
    const int c = (lane & 7) ^ (row & 7);
    asrc[j] = a.A + (long long)min(m0 + row, a.M - 1) * a.K + 8 * c;
  }
  // packed rows 2w, 2w + 1 of the step: BN / 2 lanes of 16 bytes
  const uint32_t *qsrc = a.q + (long long)(2 * wave + lane / (BN / 4)) * a.N + n0 + 4 * (lane % (BN / 4));
  // the scale row: BN / 32 lanes of 16 bytes (8 columns) per wave
  const __half *ssrc = a.s + n0 + (wave * (BN / 32) + lane) * 8;
  auto issue = [&](int u) {
    uint8_t *st = ring + (u % kS) * Cf::kStage;
    const int k0 = u * kW2BK;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(asrc[j] + k0, (CFA_LDS void *)(st + 1024 * (4 * wave + j)));
    if (lane < BN / 2)
      dma16(qsrc + (long long)(k0 / 8) * a.N, (CFA_LDS void *)(st + Cf::kABytes + wave * (8 * BN)));
    if (lane < BN / 32)
      dma16(ssrc + (long long)(k0 / a.group) * a.N,
            (CFA_LDS void *)(st + Cf::kABytes + Cf::kQBytes + wave * (BN / 32) * 16));
  };

  // dequantisation share: packed row pr, words wc .. wc + NW - 1
  const int pr = tid >> 5, wc = (tid & 31) * NW;
  // operand read offsets: A row m / B row n hold 64 k (128 bytes), chunk c
  // at position c ^ (row % 8)
  const int g = lane >> 4, col = lane & 15;
  int aoff[4][2], boff[NB][2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wm * 64 + 16 * i + col;
      aoff[i][kk] = row * 128 + (((kk * 4 + g) ^ (row & 7)) << 4);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = wn * (BN / 2) + 16 * j + col;
      boff[j][kk] = n * 128 + (((kk * 4 + g) ^ (n & 7)) << 4);
    }
  }

  f32x4 acc[4][NB];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int u = 0; u < min(kP, iters); ++u) issue(u);
  for (int it = 0; it < iters; ++it) {
    // this wave's part of stage `it` has landed and its LDS reads of step
    // it - 1 have returned; after the barrier the dequantised tile and the
    // ring slot refilled below (last read in step it - 1) are free
    w2_wait_stages<LPI, kP - 1>(min(kP - 1, iters - 1 - it));
    block_barrier();
    if (it + kP < iters) issue(it + kP);
    const uint8_t *st = ring + (it % kS) * Cf::kStage;
    {
      uint32_t w[NW];
      const uint8_t *qp = st + Cf::kABytes + pr * (BN * 4) + wc * 4;
      if (NW == 4) {
        const uint4 v = *reinterpret_cast<const uint4 *>(qp);
        w[0] = v.x; w[1] = v.y; w[2 % NW] = v.z; w[3 % NW] = v.w;
      } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(qp);
        w[0] = v.x; w[1 % NW] = v.y;
      }
      const __half *sp = reinterpret_cast<const __half *>(st + Cf::kABytes + Cf::kQBytes) + wc;
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        const float sf = __half2float(sp[j]);
        uint32_t o[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float f0 = (float)((w[j] >> (8 * p)) & 15u) * sf;
          const float f1 = (float)((w[j] >> (8 * p + 4)) & 15u) * sf;
          o[p] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f0) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f1) << 16);
        }
        const int n = wc + j;
        *reinterpret_cast<uint4 *>(btile + n * 128 + ((pr ^ (n & 7)) << 4)) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    block_barrier();  // the dequantised tile is complete
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 bfr[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) bfr[j] = *reinterpret_cast<const bf16x8 *>(btile + boff[j][kk]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x8 af = *reinterpret_cast<const bf16x8 *>(st + aoff[i][kk]);
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // C[row][col]: acc[i][j][e], row = m0 + 64 wm + 16 i + 4 g + e,
  // col = n0 + (BN / 2) wn + 16 j + lane % 16
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + wm * 64 + 16 * i + 4 * g + e;
      if (row >= a.M) continue;
      uint16_t *cr = a.C + (long long)row * a.N + n0 + wn * (BN / 2) + col;
#pragma unroll
      for (int j = 0; j < NB; ++j) cr[16 * j] = __builtin_bit_cast(uint16_t, (__bf16)acc[i][j][e]);
    }
}

}  // namespace w4
}  // namespace cfa

extern "C" int cfa_w4a16_gemm(const void *a, const uint32_t *b_quant, const void *scales, int M,
                              int N, int K, int group_size, int fp16, void *c, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (M <= 0 || N <= 0 || K <= 0) return fail_arg("M, N and K must be positive");
  if (N % 64 != 0) return fail_arg("N must be a multiple of 64");
  if (group_size <= 0 || group_size % cfa::w4::kGBK != 0 || K % group_size != 0)
    return fail_arg("group_size must be a multiple of 64 that divides K");
  if (!a || !b_quant || !scales || !c) return fail_arg("null pointer");
  if ((((uintptr_t)a | (uintptr_t)b_quant | (uintptr_t)c) & 15) != 0 || ((uintptr_t)scales & 7) != 0)
    return fail_arg("operands must be 16-byte aligned (scales 8-byte)");
  cfa::w4::GArgs g{};
  g.A = (const uint16_t *)a;
  g.q = b_quant;
  g.s = (const __half *)scales;
  g.C = (uint16_t *)c;
  g.M = M;
  g.N = N;
  g.K = K;
  g.group = group_size;
  const int cus = device_cu_count();
  // bf16 with many rows: the cooperative-dequantisation kernel
  if (!fp16 && N % 64 == 0 && group_size % cfa::w4::kW2BK == 0 && K % group_size == 0 &&
      ((uintptr_t)scales & 15) == 0 && M > 64) {
    const int mt = (M + cfa::w4::kW2BM - 1) / cfa::w4::kW2BM;
    const int bn = (N % 128 == 0 && (long long)mt * (N / 128) >= cus) ? 128 : 64;
    g.mtiles = mt;
    g.ntiles = N / bn;
    const long long blocks = (long long)mt * ((g.ntiles + 7) / 8) * 8;
    if (blocks > 0x7fffffffLL) return fail_arg("problem too large");
    hipStream_t st = (hipStream_t)stream;
    // at most one work-group per CU: spend the second one's LDS on a deeper ring
    const bool deep = blocks <= cus;
    if (bn == 128 && deep)
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4g2_kernel<128, 5>), dim3((unsigned)blocks), dim3(256), 0, st, g);
    else if (bn == 128)
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4g2_kernel<128, 3>), dim3((unsigned)blocks), dim3(256), 0, st, g);
    else if (deep)
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4g2_kernel<64, 5>), dim3((unsigned)blocks), dim3(256), 0, st, g);
    else
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4g2_kernel<64, 3>), dim3((unsigned)blocks), dim3(256), 0, st, g);
    return CFA_OK;
  }
  if (N % cfa::w4::kGBN != 0) return fail_arg("N must be a multiple of 256 (64 for bf16 with M > 64)");
  g.ntiles = N / cfa::w4::kGBN;
  const bool small = ((M + 63) / 64) * g.ntiles < cus;  // 32-row tiles fill the chip better
  const int BM = small ? 32 : 64;
  g.mtiles = (M + BM - 1) / BM;
  const long long blocks = (long long)g.mtiles * ((g.ntiles + 7) / 8) * 8;
  if (blocks > 0x7fffffffLL) return fail_arg("problem too large");
  hipStream_t st = (hipStream_t)stream;
  if (fp16) {
    if (small)
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4gemm_kernel<32, true>), dim3((unsigned)blocks), dim3(256), 0, st, g);
    else
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4gemm_kernel<64, true>), dim3((unsigned)blocks), dim3(256), 0, st, g);
  } else {
    if (small)
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4gemm_kernel<32, false>), dim3((unsigned)blocks), dim3(256), 0, st, g);
    else
      CFA_LAUNCH("w4a16_gemm", (cfa::w4::w4gemm_kernel<64, false>), dim3((unsigned)blocks), dim3(256), 0, st, g);
  }
  return CFA_OK;
}
