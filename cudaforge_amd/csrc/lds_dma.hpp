// lds_dma.hpp -- direct HBM -> LDS transfers and the waits around them.
#pragma once

#include <hip/hip_runtime.h>

#define CFA_LDS __attribute__((address_space(3)))

namespace cfa {

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, expcnt 6:4, lgkmcnt 11:8, vmcnt[5:4] in 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}

// One 16-byte-per-lane transfer HBM -> LDS: lane i's 16 bytes at `src` land at
// LDS byte address lds + 16 i.  Written as inline assembly so the compiler
// neither tracks it (its alias analysis would otherwise wait for every
// transfer before each LDS read) nor reorders it; completion is awaited with
// wait_vmcnt and published to the other waves with block_barrier.  M0 is a
// reserved register that the compiler sets right before each of its own uses,
// so overwriting it here disturbs nothing.
__device__ __forceinline__ void dma16(const void *src, CFA_LDS void *lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory");
}

// The same with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit
// byte offset: no 64-bit address arithmetic per transfer on the vector unit.
__device__ __forceinline__ void dma16_s(const void *sbase, uint32_t voff, CFA_LDS void *lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory");
}

// Work-group barrier without the release/acquire fences of __syncthreads
// (those would wait for every outstanding transfer); the empty asm statements
// keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace cfa
