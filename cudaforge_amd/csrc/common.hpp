// common.hpp -- shared helpers for the gfx950 verification kernels.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define CFA_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#define CFA_HD inline
#endif

namespace cfa {

CFA_HD uint32_t f2u(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}

CFA_HD float u2f(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

// std::max(0.0f, v) of the reference (speculative.cpp:33): (0 < v) ? v : 0.
CFA_HD float relu_ref(float v) { return (0.0f < v) ? v : 0.0f; }

// Acceptance ratio of speculative.cpp:71: q > 0 ? min(1, p / q) : 0.
CFA_HD float ratio_cpp(float p, float q) {
  if (!(q > 0.0f)) return 0.0f;
  float r = p / q;
  return (1.0f < r) ? 1.0f : r;
}

// Acceptance ratio of speculative.py:162-164: min(1, q_t / (p_d + 1e-8)).
CFA_HD float ratio_py(float q_target, float p_draft) {
  float den = p_draft + 1e-8f;
  float r = q_target / den;
  return (r > 1.0f) ? 1.0f : r;
}

}  // namespace cfa
