// dist.hpp -- a row's probabilities as the verification kernels see them.
#pragma once

#include <hip/hip_runtime.h>

// exp2(.) * invS and (v - M) * c must round exactly as written.
#pragma clang fp contract(off)

namespace cfa {

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

}  // namespace cfa
