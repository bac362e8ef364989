// seqsum.hpp -- exact, parallel replay of a left-to-right fp32 accumulation.
//
// The reference draws tokens with a sequential fp32 inverse CDF
//   cumulative = 0; for i: cumulative += probs[i]; if (r <= cumulative) return i;
// (csrc/src/scheduler/speculative.cpp:15-23) and normalises the residual with a
// sequential fp32 sum (speculative.cpp:30-35).  A tree or shuffle reduction
// rounds differently, so this file computes s_i = fl(s_{i-1} + x_i) exactly,
// for x_i >= 0, without a length-V dependency chain.
//
// Mathematics.  Cut [0, inf) into regions: region -126 is [0, 2^-125) and
// region r >= -125 is [2^r, 2^(r+1)).  Every fp32 value in region r is a
// multiple of its grid g_r = 2^(r-23), and s / g_r < 2^24.  While the running
// sum stays in region r, one step is
//     fl(s + x) = s + g_r * rne(x / g_r)
// because s is already on the grid; only an exact tie (x / g_r = n + 1/2)
// depends on s, through the parity of s / g_r (round half to even).  A result
// equal to 2^(r+1) is also exact (it is a multiple of the next grid, and any
// later non-zero step would leave the bound).  So a run of elements that stays
// in one region advances s by an integer number of grid units that is a sum
// of per-element integers -- a parallel prefix sum.  Steps that cross into a
// higher region are replayed serially with the fp32 add itself.
//
// Algorithm (one work-group per row).  Elements are staged in blocks of
// NT*16; thread t owns a tile of 16 consecutive elements.  An approximate
// prefix (exact block entry + fp32 tile sums) guesses each tile's region; the
// tile is quantised to that region's grid, giving the integer increment
// (twice: for even and odd entry parity, which differ only at ties).  One wave
// then walks the block: runs of tiles whose guess equals the region of the
// exact running sum, and whose total keeps it inside the region, are applied
// with one integer prefix sum; any other tile is replayed serially from LDS.
// Every applied increment is validated against the exact running sum, so a
// wrong guess costs time, never correctness.
#pragma once

#include "common.hpp"

namespace cfa {
namespace seq {

constexpr int kRegionMin = -126;
constexpr uint32_t kUnitsTop = 1u << 24;  // 2^(r+1) / g_r
constexpr uint32_t kSat = 1u << 25;       // saturated (certainly invalid) units
constexpr uint32_t kBad = 0xFFFFFFFFu;    // tile/wave marker: replay serially

// Region index of s >= 0 (see above).  Zero and subnormals fall in -126.
CFA_HD int region_of(float s) {
  int e = (int)((f2u(s) >> 23) & 0xff);
  return (e < 1 ? 1 : e) - 127;
}

CFA_HD float ldexp_f(float x, int e) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_ldexpf(x, e);
#else
  return ldexpf(x, e);
#endif
}

// s / g_r for s in region r (an exact integer below 2^24, or 2^24 itself).
CFA_HD uint32_t units_of(float s, int r) { return (uint32_t)ldexp_f(s, 23 - r); }

// The fp32 value a * g_r (exact for a <= 2^24).
CFA_HD float value_of(uint32_t a, int r) { return ldexp_f((float)a, r - 23); }

// Quantise x >= 0 to the grid of region r.  n = floor(x / g), with `up` set
// when the fraction is above one half and `tie` when it is exactly one half.
struct Quant {
  uint32_t n;
  uint32_t up;
  uint32_t tie;
};

CFA_HD Quant quantize(float x, int r) {
  float t = ldexp_f(x, 23 - r);
  t = (t < (float)kSat) ? t : (float)kSat;  // also maps +inf to kSat
#if defined(__HIP_DEVICE_COMPILE__)
  float fl = __builtin_floorf(t);
#else
  float fl = floorf(t);
#endif
  float f = t - fl;
  Quant q;
  q.n = (uint32_t)fl;
  q.up = (f > 0.5f) ? 1u : 0u;
  q.tie = (f == 0.5f) ? 1u : 0u;
  return q;
}

CFA_HD uint32_t sat_add(uint32_t a, uint32_t b) {
  uint32_t s = a + b;
  return (s < kSat) ? s : kSat;
}

// Integer increments of a tile of `len` elements in region r, for entry
// parity 0 (I0) and 1 (I1).  A tie rounds to the even neighbour of the
// running value, whose parity is (entry parity + increments so far) mod 2.
CFA_HD void quantize_tile(const float *x, int len, int r, uint32_t &I0, uint32_t &I1) {
  uint32_t a = 0, b = 0;
  for (int k = 0; k < len; ++k) {
    Quant q = quantize(x[k], r);
    uint32_t ia = q.n + (q.tie ? ((a + q.n) & 1u) : q.up);
    uint32_t ib = q.n + (q.tie ? ((1u + b + q.n) & 1u) : q.up);
    a = sat_add(a, ia);
    b = sat_add(b, ib);
  }
  I0 = a;
  I1 = b;
}

// Apply a run increment I (valid for the parity it was computed for) to the
// exact value s in region r; returns false when the run would leave the
// region (the caller then replays serially).
CFA_HD bool apply_units(float &s, int r, uint32_t I) {
  uint32_t a = units_of(s, r);
  if (I > kUnitsTop || a + I > kUnitsTop) return false;
  s = value_of(a + I, r);
  return true;
}

}  // namespace seq
}  // namespace cfa

#if defined(__HIPCC__)
namespace cfa {
namespace seq {

constexpr float kDelta = 1.0f / 2048.0f;  // slack on the region guess

// LDS working set of one exact pass; NT threads, 16 elements per tile.
template <int NT>
struct Shared {
  static constexpr int kTile = 16;
  static constexpr int kWaves = NT / 64;
  static constexpr int kBlock = NT * kTile;
  float x[kBlock];          // staged elements of the current block
  uint32_t tI[NT];          // tile increment (grid units) or kBad
  int16_t treg[NT];         // tile region guess
  uint32_t wI[kWaves];      // wave increment or kBad
  int16_t wreg[kWaves];     // wave region
  float wscan[kWaves];      // block scan scratch
  float s;                  // exact running value at the current block entry
  long long found;          // first index with r <= s_i, or -1
};

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

__device__ __forceinline__ float wave_incl_scan_f32(float v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    float o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Number of consecutive set bits starting at bit 0.
__device__ __forceinline__ int trailing_ones(unsigned long long m) {
  unsigned long long inv = ~m;
  return inv ? (int)__builtin_ctzll(inv) : 64;
}

// Serial replay of one 16-element tile from LDS (all lanes redundantly).
template <int NT>
__device__ long long serial_tile(const Shared<NT> &sh, int tile, float &s, bool cdf, float r,
                                 long long blk0) {
  const float *x = sh.x + tile * Shared<NT>::kTile;
  for (int k = 0; k < Shared<NT>::kTile; ++k) {
    s = s + x[k];
    if (cdf && r <= s) return blk0 + (long long)tile * Shared<NT>::kTile + k;
  }
  return -1;
}

// Walk the 64 tiles of wave w from exact value s (wave 0 executes).
template <int NT>
__device__ long long tile_sweep(const Shared<NT> &sh, int w, float &s, bool cdf, float r,
                                long long blk0) {
  const int lane = lane_id();
  int t = 0;
  while (t < 64) {
    const int rs = region_of(s);
    const uint32_t a = units_of(s, rs);
    const int ti = t + lane;
    bool vin = false;
    uint32_t I = 0;
    if (ti < 64) {
      uint32_t v = sh.tI[w * 64 + ti];
      vin = (v != kBad) && ((int)sh.treg[w * 64 + ti] == rs);
      I = vin ? v : 0u;
    }
    const uint32_t inc = wave_incl_scan_u32(I);
    const bool ok = vin && (a + inc <= kUnitsTop);
    const int nvalid = trailing_ones(__ballot(ok));
    if (cdf) {
      const bool hit = (lane < nvalid) && (r <= value_of(a + inc, rs));
      const unsigned long long hm = __ballot(hit);
      if (hm) {
        const int h = (int)__builtin_ctzll(hm);
        const uint32_t ex = __shfl(inc - I, h, 64);
        s = value_of(a + ex, rs);
        return serial_tile(sh, w * 64 + t + h, s, cdf, r, blk0);
      }
    }
    if (nvalid > 0) {
      const uint32_t tot = __shfl(inc, nvalid - 1, 64);
      s = value_of(a + tot, rs);
      t += nvalid;
      continue;
    }
    const long long f = serial_tile(sh, w * 64 + t, s, cdf, r, blk0);
    if (f >= 0) return f;
    ++t;
  }
  return -1;
}

// Walk one staged block (wave 0 executes); updates sh.s / sh.found.
template <int NT>
__device__ void sweep_block(Shared<NT> &sh, long long blk0, bool cdf, float r) {
  constexpr int NW = Shared<NT>::kWaves;
  const int lane = lane_id();
  float s = sh.s;
  long long found = -1;
  int w = 0;
  while (w < NW) {
    const int rs = region_of(s);
    const uint32_t a = units_of(s, rs);
    const int wi = w + lane;
    bool vin = false;
    uint32_t I = 0;
    if (wi < NW) {
      uint32_t v = sh.wI[wi];
      vin = (v != kBad) && ((int)sh.wreg[wi] == rs);
      I = vin ? v : 0u;
    }
    const uint32_t inc = wave_incl_scan_u32(I);
    const bool ok = vin && (a + inc <= kUnitsTop);
    const int nvalid = trailing_ones(__ballot(ok));
    if (cdf) {
      const bool hit = (lane < nvalid) && (r <= value_of(a + inc, rs));
      const unsigned long long hm = __ballot(hit);
      if (hm) {
        const int h = (int)__builtin_ctzll(hm);
        const uint32_t ex = __shfl(inc - I, h, 64);
        s = value_of(a + ex, rs);
        found = tile_sweep(sh, w + h, s, cdf, r, blk0);
        break;
      }
    }
    if (nvalid > 0) {
      const uint32_t tot = __shfl(inc, nvalid - 1, 64);
      s = value_of(a + tot, rs);
      w += nvalid;
      continue;
    }
    found = tile_sweep(sh, w, s, cdf, r, blk0);
    if (found >= 0) break;
    ++w;
  }
  if (lane == 0) {
    sh.s = s;
    if (found >= 0) sh.found = found;
  }
}

// Exact left-to-right fp32 accumulation of xf(0..n-1) (all NT threads call).
// sum mode: returns s_{n-1}.  cdf mode: *idx = first i with r <= s_i, or -1.
template <int NT, class XF>
__device__ float run(const XF &xf, long long n, bool cdf, float r, Shared<NT> &sh,
                     long long *idx) {
  constexpr int TILE = Shared<NT>::kTile;
  constexpr int BLK = Shared<NT>::kBlock;
  constexpr int NW = Shared<NT>::kWaves;
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) {
    sh.s = 0.0f;
    sh.found = -1;
  }
  __syncthreads();
  for (long long blk0 = 0; blk0 < n; blk0 += BLK) {
#pragma unroll 4
    for (int j = 0; j < TILE; ++j) {
      const int m = j * NT + tid;
      const long long i = blk0 + m;
      sh.x[m] = (i < n) ? xf(i) : 0.0f;
    }
    __syncthreads();
    const float s_blk = sh.s;
    float v[TILE];
    float A = 0.0f;
#pragma unroll
    for (int k = 0; k < TILE; ++k) {
      v[k] = sh.x[tid * TILE + k];
      A += v[k];
    }
    const float incl = wave_incl_scan_f32(A);
    if (lane == 63) sh.wscan[wave] = incl;
    __syncthreads();
    float wpre = 0.0f;
    for (int q = 0; q < wave; ++q) wpre += sh.wscan[q];
    const float E = s_blk + (wpre + (incl - A));
    const int r_lo = region_of(E * (1.0f - kDelta));
    const int r_hi = region_of((E + A) * (1.0f + kDelta));
    bool ok = (r_lo == r_hi);
    uint32_t I0 = kBad, I1 = kBad;
    if (ok) {
      quantize_tile(v, TILE, r_lo, I0, I1);
      ok = (I0 == I1) && (I0 <= kUnitsTop);
    }
    sh.tI[tid] = ok ? I0 : kBad;
    sh.treg[tid] = (int16_t)r_lo;
    const unsigned long long okm = __ballot(ok);
    const int r0 = __shfl(r_lo, 0, 64);
    const unsigned long long same = __ballot(r_lo == r0);
    const uint32_t tot = wave_sum_u32(ok ? I0 : 0u);
    if (lane == 0) {
      const bool uni = (okm == ~0ull) && (same == ~0ull);
      sh.wI[wave] = uni ? (tot < kSat ? tot : kSat) : kBad;
      sh.wreg[wave] = (int16_t)r0;
    }
    __syncthreads();
    if (wave == 0) sweep_block(sh, blk0, cdf, r);
    __syncthreads();
    if (cdf && sh.found >= 0) break;
  }
  const float out = sh.s;
  if (idx) *idx = sh.found;
  __syncthreads();
  (void)NW;
  return out;
}

}  // namespace seq
}  // namespace cfa
#endif  // __HIPCC__
