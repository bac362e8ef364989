// team.hpp -- teams of work-groups that work on one sequence together.
//
// A team is G <= 8 work-groups of one launch, all resident at once (the
// launch never holds more work-groups than the device runs together), that
// work on one sequence together.  Members
// take identical control-flow decisions from identical data, and meet at
// team barriers.  Values crossing work-groups (which may sit on different
// XCDs, whose L2s are not coherent with each other) are written with
// agent-scope atomic stores and read with agent-scope atomic loads, and every
// wave drains its stores (s_waitcnt vmcnt(0)) before its work-group arrives
// at a barrier: on gfx950 these stores write through to the device coherence
// point and are acknowledged only once performed there, and these loads
// bypass the local L2 (the argument of the split-K handoff in
// skinny_gemm.hip).  Every wait is bounded: a wait that runs out sets a
// device-wide error flag, and every later wait of the launch returns at once,
// so every wave reaches the end of the kernel.
//
// team_seq() is seq::run split over a team: member m owns elements
// [m L, (m+1) L).  In parallel the members stage and evaluate their
// segments, publish approximate segment sums, and turn their first block into
// tile / wave functions (seqsum.hpp) from the approximate entry value; a
// segment lying in one region also publishes its composed function.  Then
// every member walks the segments in order from the exact running value:
// a published function that applies (same region, no crossing, and in CDF
// mode no hit inside) advances the value at once; any other segment is
// swept exactly by its owner, which hands the exact exit value (and a CDF
// hit) to the team through a tagged word.
#pragma once

#include "seqsum.hpp"

namespace cfa {
namespace team {

constexpr int kMaxG = 8;
constexpr int kRecWords = 20;  // run-1 function (2), its region, break tile, 16 break values
constexpr long kSpinLimit = 1l << 22;   // about 0.2-0.5 s of polling

// One team's global state (part of the caller's workspace, zero before the
// launch).
struct alignas(256) State {
  unsigned long long hand[2 * (kMaxG + 1)];     // exact-pass handoffs: (tag, value), (tag, hit)
  unsigned long long pad1[32 - 2 * (kMaxG + 1)];
  // exchanged per-member values: four words (tag << 32 | value) per member,
  // in the buffer of the exchange tag's parity
  unsigned long long xw[kMaxG][2][4];
  // per member, a segment function's second run and break tile (tag << 32 |
  // value): written before an exact pass's second exchange, read after it,
  // and rewritten only after the next pass's first exchange
  unsigned long long rec[kMaxG][kRecWords];
};

// LDS a team member needs besides seq::Shared.
struct Lds {
  int failed;
  unsigned long long word;
  uint4 got[kMaxG][2];  // fetched exchange slots
};

struct Team {
  State *st;
  int *err;      // device-wide error flag
  int m, G;      // member index, members
  unsigned nb;   // exchanges done (identical in every member; tags the exchange words)
  unsigned pass; // exact passes run (tags the handoff words)
};

__device__ __forceinline__ void st32(unsigned *p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld32(unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64(unsigned long long *p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld64(unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool error_set(int *err) {
  return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void set_error(int *err) {
  __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exchange of one 16-byte value per member, which is also the team's
// barrier (every thread of every member calls it): thread 0 writes v as
// four words (tag << 32 | value) into this member's buffer of the tag's
// parity; thread j < G polls member j's four words until all carry the tag
// (a bounded wait: one that runs out sets the error flag and yields zeros),
// so l.got[j][0] = member j's value.  One round trip, where a barrier
// counter and a separate read of published values took two.  A buffer is
// written again two exchanges later: by then every member has published the
// exchange in between, which it does only after reading this one.
// The exchange in two halves: a member may publish its value, do work that
// needs nothing from the others, and collect theirs later.  It has to have
// collected an exchange before it publishes the next one.
__device__ __forceinline__ void exchange_publish(Team &t, uint4 v) {
  const unsigned tag = ++t.nb;  // the workspace starts at zero: 0 is never a tag
  __syncthreads();              // every thread is done with the previous exchange's l.got
  if (threadIdx.x == 0) {
    unsigned long long *mine = &t.st->xw[t.m][tag & 1u][0];
    const unsigned long long hi = (unsigned long long)tag << 32;
    st64(mine, hi | v.x);
    st64(mine + 1, hi | v.y);
    st64(mine + 2, hi | v.z);
    st64(mine + 3, hi | v.w);
  }
}

__device__ __forceinline__ void exchange_collect(Team &t, Lds &l) {
  const unsigned tag = t.nb;
  if (threadIdx.x < t.G) {
    unsigned long long *p = &t.st->xw[threadIdx.x][tag & 1u][0];
    unsigned long long w0 = 0, w1 = 0, w2 = 0, w3 = 0;
    long spins = 0;
    for (;;) {
      w0 = ld64(p);
      w1 = ld64(p + 1);
      w2 = ld64(p + 2);
      w3 = ld64(p + 3);
      if ((unsigned)(w0 >> 32) == tag && (unsigned)(w1 >> 32) == tag &&
          (unsigned)(w2 >> 32) == tag && (unsigned)(w3 >> 32) == tag)
        break;
      if (l.failed || ++spins > kSpinLimit || error_set(t.err)) {
        l.failed = 1;
        set_error(t.err);
        w0 = w1 = w2 = w3 = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    l.got[threadIdx.x][0] = make_uint4((uint32_t)w0, (uint32_t)w1, (uint32_t)w2, (uint32_t)w3);
  }
  __syncthreads();
}

__device__ __forceinline__ void exchange(Team &t, Lds &l, uint4 v) {
  exchange_publish(t, v);
  exchange_collect(t, l);
}
__device__ __forceinline__ uint4 f4u(float4 v) {
  return make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                    __float_as_uint(v.w));
}
__device__ __forceinline__ float4 u4f(uint4 v) {
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                     __uint_as_float(v.w));
}

// Handoff k of pass `tag`: the exact value after segment k - 1 and the CDF
// hit (-1: none), as two tagged words (thread 0 writes them).
__device__ __forceinline__ void put_hand(Team &t, int k, unsigned tag, float s, long long found) {
  if (threadIdx.x == 0) {
    st64(&t.st->hand[2 * k + 1], ((unsigned long long)tag << 32) | (uint32_t)(found + 1));
    st64(&t.st->hand[2 * k], ((unsigned long long)tag << 32) | f2u(s));
  }
}

// Waits (bounded) for handoff k of pass `tag`; every thread gets it.
__device__ __forceinline__ void get_hand(Team &t, Lds &l, int k, unsigned tag, float &s, long long &found) {
  if (threadIdx.x == 0) {
    unsigned long long v = 0, h = 0;  // failure: value 0, no hit
    if (!l.failed) {
      long spins = 0;
      for (;;) {
        v = ld64(&t.st->hand[2 * k]);
        h = ld64(&t.st->hand[2 * k + 1]);
        if ((unsigned)(v >> 32) == tag && (unsigned)(h >> 32) == tag) break;
        if (++spins > kSpinLimit || error_set(t.err)) {
          l.failed = 1;
          set_error(t.err);
          v = 0;
          h = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    l.word = ((h & 0xffffffffull) << 32) | (v & 0xffffffffull);
  }
  __syncthreads();
  const unsigned long long w = l.word;
  __syncthreads();
  s = u2f((uint32_t)(w & 0xffffffffu));
  found = (long long)(uint32_t)(w >> 32) - 1;
}

// The tile and wave functions of a block whose thread t holds the values
// v of its tile (elements 16 t .. 16 t + 15), from the entry value guess E.
// SH provides the function tables (tI, treg, wI, wreg, wserial) and wscan.
// Ends with a work-group barrier.
template <int NT, class SH>
__device__ void block_functions_v(SH &sh, const float (&v)[seq::Shared<NT>::kTile], float E) {
  using namespace seq;
  constexpr int TILE = Shared<NT>::kTile;
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float A = 0.0f;
#pragma unroll
  for (int k = 0; k < TILE; ++k) A += v[k];
  const float incl = wave_incl_scan_f32(A);
  if (lane == 63) sh.wscan[wave] = incl;
  __syncthreads();
  float wpre = 0.0f;
  for (int q = 0; q < wave; ++q) wpre += sh.wscan[q];
  const float Et = E + (wpre + (incl - A));
  int r_lo = region_of(Et * (1.0f - kDelta));
  const int r_hi = region_of((Et + A) * (1.0f + kDelta));
  bool ok = (r_lo == r_hi);
  Inc f{kBad, kBad};
  if (A == 0.0f) {
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
  const unsigned long long real = __ballot(r_lo != kAnyRegion);
  const int r0 = real ? (int)lane_bcast((uint32_t)r_lo, (int)__builtin_ctzll(real)) : kAnyRegion;
  const unsigned long long same = __ballot(r_lo == r0 || r_lo == kAnyRegion);
  const Inc wtot = wave_incl_compose(ok ? f : inc_identity());
  if (lane == 63) {
    const bool uni = (okm == ~0ull) && (same == ~0ull);
    sh.wI[wave] = uni ? wtot : Inc{kBad, kBad};
    sh.wreg[wave] = (int16_t)r0;
    sh.wserial[wave] = crossings >= kSerialCrossings ? 1 : 0;
  }
  __syncthreads();
}

// The tile and wave functions of the staged block sh.x (as seq::run) from
// the entry value guess E.  Ends with a work-group barrier.
template <int NT>
__device__ void block_functions(seq::Shared<NT> &sh, float E) {
  constexpr int TILE = seq::Shared<NT>::kTile;
  float v[TILE];
  const float4 *x4 = reinterpret_cast<const float4 *>(sh.x + threadIdx.x * TILE);
#pragma unroll
  for (int k = 0; k < TILE / 4; ++k) {
    const float4 q = x4[k];
    v[4 * k] = q.x;
    v[4 * k + 1] = q.y;
    v[4 * k + 2] = q.z;
    v[4 * k + 3] = q.w;
  }
  block_functions_v<NT>(sh, v, E);
}

// Stage elements [b0, min(b1, b0 + BLK)) of xf into sh.x (zero past the end).
template <int NT, class XF>
__device__ void stage(const XF &xf, long long b0, long long b1, seq::Shared<NT> &sh) {
  constexpr int TILE = seq::Shared<NT>::kTile;
  const int tid = (int)threadIdx.x;
  typename XF::Raw raw[TILE];
#pragma unroll
  for (int j = 0; j < TILE; ++j) {
    const long long i = b0 + (long long)j * NT + tid;
    if (i < b1) raw[j] = xf.load(i);
  }
#pragma unroll
  for (int j = 0; j < TILE; ++j) {
    const long long i = b0 + (long long)j * NT + tid;
    sh.x[j * NT + tid] = (i < b1) ? xf.eval(raw[j]) : 0.0f;
  }
  __syncthreads();
}

// fp32 sum of the staged block in a fixed order (every thread gets it).
template <int NT>
__device__ float staged_sum(seq::Shared<NT> &sh) {
  constexpr int TILE = seq::Shared<NT>::kTile;
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float4 *x4 = reinterpret_cast<const float4 *>(sh.x + tid * TILE);
  float A = 0.0f;
#pragma unroll
  for (int k = 0; k < TILE / 4; ++k) {
    const float4 q = x4[k];
    A += q.x;
    A += q.y;
    A += q.z;
    A += q.w;
  }
  const float incl = seq::wave_incl_scan_f32(A);
  if (lane == 63) sh.wscan[wave] = incl;
  __syncthreads();
  float tot = 0.0f;
  for (int q = 0; q < seq::Shared<NT>::kWaves; ++q) tot += sh.wscan[q];
  __syncthreads();
  return tot;
}

// No early exit (see team_seq).
struct NoEarlyExit {
  __device__ bool operator()(float, int) const { return false; }
};

// Exact left-to-right fp32 accumulation of xf(0 .. n-1) over the team (every
// thread of every member calls it with the same arguments).  Sum mode:
// returns s_{n-1}.  CDF mode: *idx = first i with r <= s_i, or -1.
// Sum mode only: once the members know the blocked fp32 total of the
// elements, early(total, depth) may end the pass (it returns -1): `depth`
// bounds the additions on any path of that blocked sum, so a caller that
// only needs a decision valid for every sum within the rounding bounds of
// both summation orders can skip the exact walk.
template <int NT, class XF, class Early = NoEarlyExit>
__device__ __attribute__((noinline)) float team_seq(Team &team_ref, Lds &tl, const XF &xf, long long n, bool cdf, float r,
                          seq::Shared<NT> &sh, long long *idx, Early early = Early()) {
  using namespace seq;
  constexpr int TILE = Shared<NT>::kTile;
  constexpr int BLK = Shared<NT>::kBlock;
  // a copy in registers: the caller's object is in its stack, which every
  // store through a generic pointer could alias (each use would reload it)
  Team tm = team_ref;
  const int tid = (int)threadIdx.x, wave = tid >> 6;
  const unsigned tag = ++tm.pass;  // the workspace starts at zero: 0 is never a tag
  const long long L = ((n + tm.G - 1) / tm.G + TILE - 1) / TILE * TILE;
  const long long lo = min(n, (long long)tm.m * L), hi = min(n, lo + L);
  const bool multi = (hi - lo) > BLK;

  // A: stage the segment's first block; approximate segment sum
  stage<NT>(xf, lo, min(hi, lo + BLK), sh);
  float T = staged_sum<NT>(sh);
  for (long long b0 = lo + BLK; b0 < hi; b0 += BLK) {  // later blocks: sum only
    float part = 0.0f;
    for (int j = 0; j < TILE; ++j) {
      const long long i = b0 + (long long)j * NT + tid;
      if (i < hi) part += xf.eval(xf.load(i));
    }
    const float incl = wave_incl_scan_f32(part);
    if ((tid & 63) == 63) sh.wscan[wave] = incl;
    __syncthreads();
    for (int q = 0; q < Shared<NT>::kWaves; ++q) T += sh.wscan[q];
    __syncthreads();
  }
  exchange(tm, tl, make_uint4(f2u(T), 0u, 0u, 0u));
  float E = 0.0f;
  for (int j = 0; j < tm.m; ++j) E += u2f(tl.got[j][0].x);
  if (!cdf) {
    float tot = 0.0f;
    for (int j = 0; j < tm.G; ++j) tot += u2f(tl.got[j][0].x);
    // per member: 16 sequential adds per thread, a 6-level wave scan and
    // 16 waves, per block; then the blocks and the G members
    const long long blocks = (L + BLK - 1) / BLK;
    const int depth = (int)(blocks * (16 + 6 + 16 + 1)) + tm.G;
    if (early(tot, depth)) {
      if (idx) *idx = -1;
      __syncthreads();
      team_ref.nb = tm.nb;
      team_ref.pass = tm.pass;
      return -1.0f;
    }
  }

  // B: tile / wave functions of the first block from the guess E; the
  // segment's composed function when it lies in one region
  block_functions<NT>(sh, E);
  if (tid == 0) {
    Inc F = inc_identity();
    int reg = kAnyRegion;
    bool valid = !multi;
    for (int w = 0; w < Shared<NT>::kWaves && valid; ++w) {
      const Inc wi = sh.wI[w];
      const int wr = sh.wreg[w];
      if (wi.e == kBad) {
        valid = false;
      } else if (wr != kAnyRegion) {
        if (reg == kAnyRegion)
          reg = wr;
        else if (reg != wr)
          valid = false;
        F = compose(F, wi);
      }
    }
    tl.got[0][1] = make_uint4(F.e, F.o, (uint32_t)reg, valid ? 1u : 0u);  // scratch
  }
  __syncthreads();
  exchange(tm, tl, tl.got[0][1]);

  // C: walk the segments from the exact running value
  float s = 0.0f;
  long long found = -1;
  for (int j = 0; j < tm.G; ++j) {
    const uint4 fj = tl.got[j][0];
    bool applies = false;
    float snext = s;
    if (fj.w) {
      const int reg = (int)fj.z;
      if (reg == kAnyRegion) {
        applies = true;
      } else {
        const int rs = region_of(s);
        if (rs == reg) {
          const uint32_t a = units_of(s, rs);
          const uint32_t inc = inc_at(Inc{fj.x, fj.y}, a);
          if (a + inc <= kUnitsTop) {
            applies = true;
            snext = value_of(a + inc, rs);
          }
        }
      }
    }
    if (applies && !(cdf && r <= snext)) {
      s = snext;
      continue;
    }
    if (j == tm.m) {  // sweep this segment exactly from s
      if (tid == 0) {
        sh.s = s;
        sh.found = -1;
      }
      __syncthreads();
      if (wave == 0) sweep_block(sh, lo, cdf, r);
      __syncthreads();
      for (long long b0 = lo + BLK; b0 < hi && !(cdf && sh.found >= 0); b0 += BLK) {
        stage<NT>(xf, b0, min(hi, b0 + BLK), sh);
        block_functions<NT>(sh, sh.s);
        if (wave == 0) sweep_block(sh, b0, cdf, r);
        __syncthreads();
      }
      s = sh.s;
      found = sh.found;
      put_hand(tm, j + 1, tag, s, found);
      __syncthreads();
    } else {
      get_hand(tm, tl, j + 1, tag, s, found);
    }
    if (cdf && found >= 0) break;
  }
  if (idx) *idx = found;
  __syncthreads();
  team_ref.nb = tm.nb;
  team_ref.pass = tm.pass;
  return s;
}

}  // namespace team
}  // namespace cfa
