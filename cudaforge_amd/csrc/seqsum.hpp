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
// tile is quantised to that region's grid, giving its integer increment for
// an even and for an odd entry parity (they differ only through ties).  A
// tile is thus a function parity -> increment; the exit parity follows from
// the increment, so two tiles compose into one such function (an associative
// operation, `compose`).  One wave then walks the block: runs of tiles whose
// guess equals the region of the exact running sum, and whose composed
// increment keeps it inside the region, are applied with one composition
// scan; any other tile is replayed serially.  Every applied increment is
// validated against the exact running sum, so a wrong guess costs time,
// never correctness.
#pragma once

#include "common.hpp"

namespace cfa {
namespace seq {

constexpr int kRegionMin = -126;
constexpr uint32_t kUnitsTop = 1u << 24;  // 2^(r+1) / g_r
constexpr uint32_t kSat = 1u << 25;       // saturated (certainly invalid) units
constexpr uint32_t kBad = 0xFFFFFFFFu;    // tile/wave marker: replay serially
constexpr int kAnyRegion = 0x7fff;        // an all-zero tile fits every region
// Slack on the region guess.  The guess need not be rigorous (the walk checks
// every applied increment against the exact running value); the slack only
// trades guesses near a power of two for serial replays.
constexpr float kDelta = 1.0f / 65536.0f;
// Tiles straddling a region boundary from which a wave is replayed as one
// serial run instead of tile by tile: a crossing costs the tile-level walk
// about 2K cycles, a serial replay of the wave's 1024 elements about 5K.
constexpr int kSerialCrossings = 3;

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

// Fast path of quantize_tile: when no element of the tile is an exact tie
// (x / g_r = n + 1/2), both parities add the same sum of round-to-nearest
// integers.  Returns false if some element is a tie (use quantize_tile).
CFA_HD bool quantize_tile_fast(const float *x, int len, int r, uint32_t &I) {
  uint32_t acc = 0;
  bool tie = false;
  for (int k = 0; k < len; ++k) {
    float t = ldexp_f(x[k], 23 - r);
    t = (t < (float)kSat) ? t : (float)kSat;
#if defined(__HIP_DEVICE_COMPILE__)
    const float n = __builtin_rintf(t);
    tie |= (__builtin_fabsf(t - n) == 0.5f);
#else
    const float n = rintf(t);
    tie |= (fabsf(t - n) == 0.5f);
#endif
    acc = sat_add(acc, (uint32_t)n);
  }
  I = acc;
  return !tie;
}

// A run of elements inside one region as a function of the entry parity:
// e / o = grid units added when the running value enters with an even / odd
// unit count.  e == kBad marks an invalid run.
struct Inc {
  uint32_t e, o;
};

CFA_HD Inc inc_identity() { return Inc{0u, 0u}; }

// A then B: B sees the parity A leaves behind.
CFA_HD Inc compose(Inc A, Inc B) {
  Inc C;
  C.e = sat_add(A.e, (A.e & 1u) ? B.o : B.e);
  C.o = sat_add(A.o, ((1u + A.o) & 1u) ? B.o : B.e);
  return C;
}

// Units added by f when entered at unit count a.
CFA_HD uint32_t inc_at(Inc f, uint32_t a) { return (a & 1u) ? f.o : f.e; }

}  // namespace seq
}  // namespace cfa

#if defined(__HIPCC__)
namespace cfa {
namespace seq {


// LDS working set of one exact pass; NT threads, 16 elements per tile.
template <int NT>
struct Shared {
  static constexpr int kTile = 16;
  static constexpr int kWaves = NT / 64;
  static constexpr int kBlock = NT * kTile;
  alignas(16) float x[kBlock];  // staged elements of the current block
  Inc tI[NT];                   // tile function (e == kBad: replay serially)
  int16_t treg[NT];             // tile region guess
  Inc wI[kWaves];               // wave function or kBad
  int16_t wreg[kWaves];         // wave region
  uint8_t wserial[kWaves];      // the wave crosses several regions: replay it serially
  float wscan[kWaves];          // block scan scratch
  float s;                      // exact running value at the current block entry
  long long found;              // first index with r <= s_i, or -1
};

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// DPP lane moves (GFX9 encodings): row_shr:n shifts within rows of 16 lanes
// (zero-filled), row_bcast:15 / :31 broadcast lane 15 / 31 of a row to the
// rows selected by the row mask.  A disabled or out-of-row lane reads 0,
// which is the identity of both scans below.
constexpr int kDppRowShr = 0x110;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xf, true);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ Inc dpp_inc(Inc v) {
  return Inc{dpp_u32<CTRL, ROWMASK>(v.e), dpp_u32<CTRL, ROWMASK>(v.o)};
}

// Inclusive scan of tile functions across the wave in lane order (DPP:
// Hillis-Steele inside rows of 16, then the row carries).
__device__ __forceinline__ Inc wave_incl_compose(Inc v) {
  v = compose(dpp_inc<kDppRowShr | 1, 0xf>(v), v);
  v = compose(dpp_inc<kDppRowShr | 2, 0xf>(v), v);
  v = compose(dpp_inc<kDppRowShr | 4, 0xf>(v), v);
  v = compose(dpp_inc<kDppRowShr | 8, 0xf>(v), v);
  v = compose(dpp_inc<kDppRowBcast15, 0xa>(v), v);
  v = compose(dpp_inc<kDppRowBcast31, 0xc>(v), v);
  return v;
}

// Inclusive integer prefix sum across the wave (same DPP pattern); the
// inputs here are at most 2^25 each, so 64 of them cannot overflow.
__device__ __forceinline__ uint32_t wave_incl_add_u32(uint32_t v) {
  v += dpp_u32<kDppRowShr | 1, 0xf>(v);
  v += dpp_u32<kDppRowShr | 2, 0xf>(v);
  v += dpp_u32<kDppRowShr | 4, 0xf>(v);
  v += dpp_u32<kDppRowShr | 8, 0xf>(v);
  v += dpp_u32<kDppRowBcast15, 0xa>(v);
  v += dpp_u32<kDppRowBcast31, 0xc>(v);
  return v;
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL, ROWMASK>(__float_as_uint(v)));
}

// Inclusive fp32 prefix sum across the wave (same DPP pattern; 0.0f is the
// zero fill).
__device__ __forceinline__ float wave_incl_scan_f32(float v) {
  v += dpp_f32<kDppRowShr | 1, 0xf>(v);
  v += dpp_f32<kDppRowShr | 2, 0xf>(v);
  v += dpp_f32<kDppRowShr | 4, 0xf>(v);
  v += dpp_f32<kDppRowShr | 8, 0xf>(v);
  v += dpp_f32<kDppRowBcast15, 0xa>(v);
  v += dpp_f32<kDppRowBcast31, 0xc>(v);
  return v;
}

// Value of v in lane `src` (wave-uniform src).
__device__ __forceinline__ uint32_t lane_bcast(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, src);
}

// Number of consecutive set bits starting at bit 0.
__device__ __forceinline__ int trailing_ones(unsigned long long m) {
  unsigned long long inv = ~m;
  return inv ? (int)__builtin_ctzll(inv) : 64;
}

// The reference's sequential fp32 adds of 16 values x >= 0 to s and, in CDF
// mode, the first k with r <= the running value after x[k] (-1: none).  The
// adds form one dependent chain with nothing else on it; the running value
// never decreases, so the hit is searched only when the last partial sum
// reaches r (static indices: a dynamically indexed array would live in
// scratch).
__device__ __forceinline__ int replay16(const float (&x)[16], float &s, bool cdf, float r) {
  float ps[16];
  float acc = s;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    acc = acc + x[k];
    ps[k] = acc;
  }
  if (cdf && r <= acc) {
    int k = 15;
    float sk = ps[15];
#pragma unroll
    for (int q = 14; q >= 0; --q) {
      const bool h = r <= ps[q];
      k = h ? q : k;
      sk = h ? ps[q] : sk;
    }
    s = sk;
    return k;
  }
  s = acc;
  return -1;
}

// Serial replay of one 16-element tile (all lanes redundantly; the four
// 16-byte LDS reads are broadcasts and are issued before the dependent adds).
template <int NT>
__device__ long long serial_tile(const Shared<NT> &sh, int tile, float &s, bool cdf, float r,
                                 long long blk0) {
  const float4 *x4 = reinterpret_cast<const float4 *>(sh.x + tile * Shared<NT>::kTile);
  float x[16];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 q = x4[k];
    x[4 * k] = q.x;
    x[4 * k + 1] = q.y;
    x[4 * k + 2] = q.z;
    x[4 * k + 3] = q.w;
  }
  const int k = replay16(x, s, cdf, r);
  return k < 0 ? -1 : blk0 + (long long)tile * Shared<NT>::kTile + k;
}

// Walk `count` items (tiles of one wave, or the waves of a block) from the
// exact value s.  item(i) returns (function, region guess); descend(i, s)
// replays item i exactly from s (updating s) and returns a CDF hit or -1.
template <class Item, class Descend>
__device__ long long walk(int count, float &s, bool cdf, float r, const Item &item,
                          const Descend &descend) {
  const int lane = lane_id();
  int t = 0;
  while (t < count) {
    const int rs = region_of(s);
    const uint32_t a = units_of(s, rs);
    const int ti = t + lane;
    bool vin = false, none = false;
    Inc f = inc_identity();
    if (ti < count) {
      int reg;
      const Inc v = item(ti, reg);
      none = (v.e == kBad);
      vin = !none && (reg == rs || reg == kAnyRegion);
      if (vin) f = v;
    }
    const unsigned long long nonem = __ballot(none);
    // Without a tie-dependent item the functions are plain integers: an add
    // scan (6 DPP adds) replaces the composition scan.
    uint32_t inc;
    if (__ballot(f.e != f.o) == 0ull)
      inc = wave_incl_add_u32(f.e);
    else
      inc = inc_at(wave_incl_compose(f), a);
    const bool ok = vin && (a + inc <= kUnitsTop);
    const int nvalid = trailing_ones(__ballot(ok));
    if (cdf) {
      const bool hit = (lane < nvalid) && (r <= value_of(a + inc, rs));
      const unsigned long long hm = __ballot(hit);
      if (hm) {
        const int h = (int)__builtin_ctzll(hm);
        const uint32_t prev = lane_bcast(inc, h > 0 ? h - 1 : 0);
        s = value_of(a + (h > 0 ? prev : 0u), rs);
        return descend(t + h, s);
      }
    }
    if (nvalid > 0) {
      const uint32_t tot = lane_bcast(inc, nvalid - 1);
      s = value_of(a + tot, rs);
      t += nvalid;
      // an item without a function that ends the run is replayed right away
      // (one descend call site: the replay is inlined once)
      if (nvalid == 64 || ((nonem >> nvalid) & 1ull) == 0ull || t >= count) continue;
    }
    const long long f2 = descend(t, s);
    if (f2 >= 0) return f2;
    ++t;
  }
  return -1;
}

// Serial replay of the 1024 values xs[0 .. 1023] of elements i0 .. (all
// lanes redundantly; the 16-byte LDS reads are broadcasts, eight of them in
// flight ahead of the adds).
__device__ __forceinline__ long long serial_run1024(const float *xs, long long i0, float &s,
                                                    bool cdf, float r) {
  constexpr int kElems = 1024;
  const float4 *x4 = reinterpret_cast<const float4 *>(xs);
  float acc = s;
  for (int c = 0; c < kElems / 4; c += 8) {
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = x4[c + j];
    float ps[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc = acc + v[j].x;
      ps[4 * j] = acc;
      acc = acc + v[j].y;
      ps[4 * j + 1] = acc;
      acc = acc + v[j].z;
      ps[4 * j + 2] = acc;
      acc = acc + v[j].w;
      ps[4 * j + 3] = acc;
    }
    if (cdf && r <= acc) {
      // the first hit of this batch (static indices: no scratch array)
      int k = 31;
      float sk = ps[31];
#pragma unroll
      for (int q = 30; q >= 0; --q) {
        const bool h = r <= ps[q];
        k = h ? q : k;
        sk = h ? ps[q] : sk;
      }
      s = sk;
      return i0 + 4 * c + k;
    }
  }
  s = acc;
  return -1;
}

// Serial replay of wave w's 64 tiles of the staged block.
template <int NT>
__device__ long long serial_wave(const Shared<NT> &sh, int w, float &s, bool cdf, float r,
                                 long long blk0) {
  constexpr int kElems = 64 * Shared<NT>::kTile;
  static_assert(kElems == 1024, "a wave's span is 1024 elements");
  return serial_run1024(sh.x + w * kElems, blk0 + (long long)w * kElems, s, cdf, r);
}

// Walk one staged block (wave 0 executes); updates sh.s / sh.found.
template <int NT>
__device__ void sweep_block(Shared<NT> &sh, long long blk0, bool cdf, float r) {
  constexpr int NW = Shared<NT>::kWaves;
  float s = sh.s;
  auto tile_desc = [&](int w) {
    return [&sh, w, cdf, r, blk0](int i, float &ss) -> long long {
      return serial_tile(sh, w * 64 + i, ss, cdf, r, blk0);
    };
  };
  auto wave_item = [&sh](int i, int &reg) -> Inc {
    reg = sh.wreg[i];
    return sh.wI[i];
  };
  auto wave_desc = [&](int w, float &ss) -> long long {
    if (sh.wserial[w]) return serial_wave(sh, w, ss, cdf, r, blk0);
    auto tile_item = [&sh, w](int i, int &reg) -> Inc {
      reg = sh.treg[w * 64 + i];
      return sh.tI[w * 64 + i];
    };
    return walk(64, ss, cdf, r, tile_item, tile_desc(w));
  };
  const long long found = walk(NW, s, cdf, r, wave_item, wave_desc);
  if (lane_id() == 0) {
    sh.s = s;
    if (found >= 0) sh.found = found;
  }
}

// Exact left-to-right fp32 accumulation of xf(0..n-1) (all NT threads call).
// sum mode: returns s_{n-1}.  cdf mode: *idx = first i with r <= s_i, or -1.
// XF provides Raw load(i) (memory only) and float eval(Raw): the loads of
// block k+1 are issued before block k is swept and evaluated only at the top
// of the next iteration, so memory latency overlaps the serial sweep.
template <int NT, class XF>
__device__ float run(const XF &xf, long long n, bool cdf, float r, Shared<NT> &sh,
                     long long *idx) {
  constexpr int TILE = Shared<NT>::kTile;
  constexpr int BLK = Shared<NT>::kBlock;
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) {
    sh.s = 0.0f;
    sh.found = -1;
  }
  typename XF::Raw raw[TILE];
#pragma unroll
  for (int j = 0; j < TILE; ++j) {
    const long long i = (long long)j * NT + tid;
    if (i < n) raw[j] = xf.load(i);
  }
  __syncthreads();
  for (long long blk0 = 0; blk0 < n; blk0 += BLK) {
#pragma unroll
    for (int j = 0; j < TILE; ++j) {
      const int m = j * NT + tid;
      sh.x[m] = (blk0 + m < n) ? xf.eval(raw[j]) : 0.0f;
    }
    __syncthreads();
    const long long nb = blk0 + BLK;
    if (nb < n) {
#pragma unroll
      for (int j = 0; j < TILE; ++j) {
        const long long i = nb + (long long)j * NT + tid;
        if (i < n) raw[j] = xf.load(i);
      }
    }
    const float s_blk = sh.s;
    float v[TILE];
    const float4 *x4 = reinterpret_cast<const float4 *>(sh.x + tid * TILE);
#pragma unroll
    for (int k = 0; k < TILE / 4; ++k) {
      const float4 q = x4[k];
      v[4 * k] = q.x;
      v[4 * k + 1] = q.y;
      v[4 * k + 2] = q.z;
      v[4 * k + 3] = q.w;
    }
    float A = 0.0f;
#pragma unroll
    for (int k = 0; k < TILE; ++k) A += v[k];
    const float incl = wave_incl_scan_f32(A);
    if (lane == 63) sh.wscan[wave] = incl;
    __syncthreads();
    float wpre = 0.0f;
    for (int q = 0; q < wave; ++q) wpre += sh.wscan[q];
    const float E = s_blk + (wpre + (incl - A));
    int r_lo = region_of(E * (1.0f - kDelta));
    const int r_hi = region_of((E + A) * (1.0f + kDelta));
    bool ok = (r_lo == r_hi);
    Inc f{kBad, kBad};
    if (A == 0.0f) {  // x >= 0: every element is zero, the identity in any region
      ok = true;
      r_lo = kAnyRegion;
      f = inc_identity();
    } else if (ok) {
      uint32_t I;
      if (quantize_tile_fast(v, TILE, r_lo, I))
        f = Inc{I, I};
      else
        quantize_tile(v, TILE, r_lo, f.e, f.o);
      ok = (f.e <= kUnitsTop) && (f.o <= kUnitsTop);
      if (!ok) f = Inc{kBad, kBad};
    }
    sh.tI[tid] = f;
    sh.treg[tid] = (int16_t)r_lo;
    const unsigned long long okm = __ballot(ok);
    const int crossings = __popcll(__ballot(!ok && A != 0.0f));
    // the wave's region: that of its first tile with a region (all-zero waves: any)
    const unsigned long long real = __ballot(r_lo != kAnyRegion);
    const int r0 = real ? (int)seq::lane_bcast((uint32_t)r_lo, (int)__builtin_ctzll(real)) : kAnyRegion;
    const unsigned long long same = __ballot(r_lo == r0 || r_lo == kAnyRegion);
    const Inc wtot = wave_incl_compose(ok ? f : inc_identity());
    if (lane == 63) {
      const bool uni = (okm == ~0ull) && (same == ~0ull);
      sh.wI[wave] = uni ? wtot : Inc{kBad, kBad};
      sh.wreg[wave] = (int16_t)r0;
      sh.wserial[wave] = crossings >= kSerialCrossings ? 1 : 0;
    }
    __syncthreads();
    if (wave == 0) sweep_block(sh, blk0, cdf, r);
    __syncthreads();
    if (cdf && sh.found >= 0) break;
  }
  const float out = sh.s;
  if (idx) *idx = sh.found;
  __syncthreads();
  return out;
}

}  // namespace seq
}  // namespace cfa
#endif  // __HIPCC__
