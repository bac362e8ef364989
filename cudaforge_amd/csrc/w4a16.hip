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

}  // namespace w4
}  // namespace cfa

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
