// silu.hpp -- the SiLU gate of a Llama FFN, rounded the same way by every
// kernel of this library that forms it (cfa_silu_mul and the SiLU-gated GEMM
// epilogues), so that a fused epilogue gives the bits of the product followed
// by cfa_silu_mul: g and u rounded to bf16, s = bf16(g / (1 + e^-g)), out =
// bf16(s * u), round to nearest even.
//
// e^-g is exp2(-g log2 e) on the hardware exponential and the quotient is g
// times the hardware reciprocal, each within about one fp32 ulp: far below
// the bf16 rounding that follows, and about five instructions against some
// thirty for the library exp and an IEEE division (at the 8B target's
// 504 x 14336 features that difference was 11 us of VALU work per call).
// Large negative g: e^-g = inf, reciprocal 0, s = -0; large positive g:
// e^-g = 0, s = g.  The bf16 roundings are the hardware conversion of
// packed pairs, so pairs of features share each conversion.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace cfa {

typedef float silu_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 silu_bf16x2 __attribute__((ext_vector_type(2)));

// two fp32 values to a packed bf16 pair (one conversion instruction)
__device__ __forceinline__ uint32_t silu_pk(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(silu_f32x2{a, b}, silu_bf16x2));
}
__device__ __forceinline__ float silu_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float silu_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// Two features at once from fp32 gate and up values (a GEMM's sums, or
// bf16 values widened): the packed pair bf16(bf16(silu(g)) * u), low half
// feature 0.
__device__ __forceinline__ uint32_t silu_gate2(float g0, float u0, float g1, float u1) {
  const uint32_t gp = silu_pk(g0, g1), up = silu_pk(u0, u1);
  const uint32_t sp = silu_pk(silu_f32(silu_lo(gp)), silu_f32(silu_hi(gp)));
  return silu_pk(silu_lo(sp) * silu_lo(up), silu_hi(sp) * silu_hi(up));
}

// one feature: the low half of the pair form
__device__ __forceinline__ uint16_t silu_gate(float g, float u) {
  return (uint16_t)silu_gate2(g, u, 0.0f, 0.0f);
}

}  // namespace cfa
