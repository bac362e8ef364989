// tree_attention.hip -- tree-masked verification attention over a paged KV
// cache, bf16 MFMA for gfx950.
//
// For sequence b, KV head h and the G = Hq / Hkv query heads sharing it, the
// N draft-tree nodes attend to every context token [0, ctx_b) and to the tree
// tokens ctx_b + j of their ancestors-or-self j (bit j of the node's ancestor
// mask).  K and V live in a paged pool laid out as
//   pool[block][layer][kv_head][slot][head_dim]  (bf16)
// -- the per-block layer stride of csrc/src/memory/paged_kv_cache.cpp:13-21
// and the block addressing of :409-421 -- and the tree's own K/V have already
// been appended at positions ctx_b .. ctx_b + N - 1.  The queries are the
// nodes first_node .. N - 1 (all of them for a verify step; the newest tree
// level for a draft model growing its tree).  head_dim is 128 or 64 (a
// template parameter).
//
// One work-group = (split, kv head, sequence); its 8 waves hold all the
// G * (N - first_node) query rows (two 16-row tiles each, Q^T in registers, pre-scaled by
// scale*log2(e)).  64-key K and V tiles move HBM -> LDS with direct 16-byte
// global_load_lds transfers (no register staging) into two rings (K: 4
// stages, V: 5), three tiles ahead of the tile being computed; the split's
// page lookups are resolved once into an LDS table.  Everything is computed
// in the transposed form
//   S^T = K Q^T - b        (MFMA A = K rows, B = Q^T columns, C = -b)
//   O^T += V^T P^T         (MFMA A = V^T rows, B = P^T columns)
//   l   += 1^T P^T         (row sums on the MFMA unit too)
// so each lane owns one query column throughout: the softmax of a column and
// the rescale of its O^T column stay in registers, and the P^T operand of the
// second product is exp2 of the first product's output in bf16.  Within a
// 32-key block the two 16-key MFMA tiles take keys {8g+i} and {8g+4+i}
// (g = lane / 16, i < 4), so lane (g, q) ends up with keys 8g..8g+7 of
// column q: exactly its 8-element k-slice of P^T.  The matching V^T k-slice
// comes from two ds_read_b64_tr_b16 transposed reads of the V tile, which
// stays in its natural [key][d] layout.
//
// Each tile runs as a VALU phase (mask, column maxima, exponentials) and an
// MFMA phase (PV of this tile, QK of the next).  Waves w and w + 4 share a
// SIMD and run one phase apart, so one's exponentials overlap the other's
// MFMAs.
//
// LDS layouts (2 * head_dim-byte rows, 16-byte chunks XOR-swizzled so that
// the MFMA operand reads of one wave hit distinct banks; k_swz / v_swz):
//   K: row R holds key 32*(R/32) + 8*((R/4)%4) + 4*((R/16)%2) + R%4 (each
//      16-row MFMA tile reads consecutive rows).
//   V: row = key.
//
// Softmax rescaling is lazy: a column's exponent base b only moves when its
// running maximum exceeds it by more than kRescaleSlack (log2 units), so P^T
// entries stay below 2^kRescaleSlack and the O^T rescale is rare.  Splits of
// the key range write normalised bf16 partials with their (base, sum), merged
// by a log-sum-exp pass.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "abi_internal.hpp"
#include "lds_dma.hpp"


namespace cfa {
namespace tree {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kKT = 64;                       // keys per tile
constexpr int kWaves = 8;
constexpr int kNT = kWaves * 64;              // threads per work-group
constexpr int kQT = 2;                        // 16-row query tiles per wave
constexpr int kMaxRows = kWaves * kQT * 16;   // 256 query rows per work-group
constexpr int kKStages = 4;                   // K-tile ring (tile u: stage u % 4)
constexpr int kVStages = 5;                   // V-tile ring (read one iteration after K)
constexpr float kRescaleSlack = 8.0f;         // log2 units

// Layout constants of head size D (64 or 128): K / V rows of D bf16 values,
// D / 8 16-byte chunks each.
template <int D>
struct Geo {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static constexpr int kRowBytes = D * 2;             // one K or V row
  static constexpr int kTileBytes = kKT * kRowBytes;  // 8 or 16 KiB
  static constexpr int kChunks = D / 8;               // 16-byte chunks per row
  static constexpr int kRowsPerLoad = 1024 / kRowBytes;  // rows per 1 KiB transfer
  static constexpr int kLoadsPerTile = 2 * (8 / kRowsPerLoad);  // K + V transfers per wave
  static constexpr int kKK = D / 32;                  // k-slices of the QK product
  static constexpr int kDT = D / 16;                  // 16-row blocks of O^T
  static constexpr int kMfma = 2 * kDT * kQT + 2 * kQT + 4 * kKK * kQT;  // per MFMA phase
};
#ifndef CFA_TA_SGB
#define CFA_TA_SGB 1
#endif
constexpr int kMaxGroups = 1024;              // 16-key groups per split (page lookup table)
constexpr int kMaxTilesPerSplit = kMaxGroups / (kKT / 16);

struct Args {
  const uint16_t *q;       // [B, Nq, Hq, D]
  const uint16_t *kpool;   // [blocks, layers, Hkv, bs, D]
  const uint16_t *vpool;
  const int32_t *bt;       // [B, max_blocks]
  const int32_t *ctx;      // [B]
  const uint64_t *mask;    // [N] or [B, N]
  long long mask_sb;
  uint16_t *out;           // [B, Nq, Hq, D]
  uint16_t *part_o;        // [S, B, Hkv, rows, D] partial outputs O / l, bf16
  float2 *part_ml;         // [S, B, Hkv, rows] (exponent base in log2 units, sum)
  int B, N, Hq, Hkv, G, rows;
  int q0, Nq;              // query nodes q0 .. N - 1 (Nq = N - q0 of them)
  int max_blocks, num_blocks, num_layers, layer, bs;
  int splits, tiles_per_split;
  float scale_log2;        // sm_scale * log2(e)
};

__device__ __forceinline__ uint4 ld_g16(const uint16_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}

// Key (tile-relative) held by K-tile LDS row R.
__device__ __forceinline__ int k_key_of_row(int R) {
  return (R & ~31) + ((R >> 2) & 3) * 8 + ((R >> 4) & 1) * 4 + (R & 3);
}

// LDS swizzles (16-byte chunk c of a row sits at position c ^ swizzle):
//   K-tile row R:  D = 128: R % 16;  D = 64: (R / 2) % 8.  A 16-row MFMA
//     operand read then touches every bank once per 16 lanes.
//   V-tile row key: twice the 32-byte block swizzle vh, the same for keys k
//     and k + 4 (one transposed-read pair); D = 128: (key % 4) | 4 ((key / 8)
//     % 2); D = 64: ((key / 2) % 2) | 2 ((key / 8) % 2).  The four rows of one
//     transposed read then land in distinct banks.
template <int D>
__device__ __forceinline__ int k_swz(int R) {
  return D == 128 ? (R & 15) : ((R >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int v_swz(int key) {
  return D == 128 ? (((key & 3) | ((key >> 1) & 4)) << 1) : ((((key >> 1) & 1) | ((key >> 2) & 2)) << 1);
}

// Pool element offset of the row holding position gstart = min(16 gi,
// nkeys - 1), the first row 16-key group gi reads.  Page index and block id
// are clamped into the table and the pool, so a corrupt table can never send
// a load outside the pool.
template <int D>
__device__ __forceinline__ long long group_row_offset(const Args &a, const int32_t *btb, int gi,
                                                      int nkeys, int h) {
  const int gstart = min(gi * 16, nkeys - 1);
  const int page = min(gstart / a.bs, a.max_blocks - 1);
  const int blk = min(max(btb[page], 0), a.num_blocks - 1);
  return (((long long)blk * a.num_layers + a.layer) * a.Hkv + h) * (long long)(a.bs * D) +
         (long long)(gstart - page * a.bs) * D;
}

__device__ __forceinline__ long long uniform_i64(long long v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((unsigned long long)v >> 32));
  return (long long)(((unsigned long long)hi << 32) | lo);
}

// Issue this wave's share of the tile at key kbase: K-tile LDS rows 8w..8w+7
// and V keys 8w..8w+7, in 1 KiB transfers of 1024 / (2 D) rows.  Each
// transfer stays inside one 16-key group, and a group never straddles a page
// (block_size % 16 == 0).  Keys at or past nkeys re-read key nkeys - 1: a
// finite, in-bounds row that the mask then hides.  gtab holds the split's
// group row offsets (group_row_offset) from group g0 on.
template <int D>
__device__ __forceinline__ void issue_tile(const Args &a, const long long *gtab, int g0, int kbase,
                                           int nkeys, uint8_t *kdst, uint8_t *vdst, int wave,
                                           int lane) {
  using Gm = Geo<D>;
  constexpr int RPL = Gm::kRowsPerLoad;
  const int sub = lane / Gm::kChunks, pc = lane % Gm::kChunks;
  {
    // K: the wave's rows hold keys of the tile's 16-group 2 (w / 4) + (w % 2)
    const int gi = kbase / 16 + 2 * (wave >> 2) + (wave & 1);
    const int gstart = min(gi * 16, nkeys - 1);
    const uint16_t *base = a.kpool + uniform_i64(gtab[gi - g0]);
#pragma unroll
    for (int j = 0; j < 8 / RPL; ++j) {
      const int R = 8 * wave + RPL * j + sub;
      const int c = pc ^ k_swz<D>(R);
      const int pos = min(kbase + k_key_of_row(R), nkeys - 1);
      dma16(base + ((pos - gstart) * D + c * 8),
            (CFA_LDS void *)(kdst + (8 * wave + RPL * j) * Gm::kRowBytes));
    }
  }
  {
    // V: keys 8w..8w+7, in the tile's 16-group w / 2
    const int gi = kbase / 16 + (wave >> 1);
    const int gstart = min(gi * 16, nkeys - 1);
    const uint16_t *base = a.vpool + uniform_i64(gtab[gi - g0]);
#pragma unroll
    for (int j = 0; j < 8 / RPL; ++j) {
      const int key = 8 * wave + RPL * j + sub;
      const int c = pc ^ v_swz<D>(key);
      const int pos = min(kbase + key, nkeys - 1);
      dma16(base + ((pos - gstart) * D + c * 8),
            (CFA_LDS void *)(vdst + (8 * wave + RPL * j) * Gm::kRowBytes));
    }
  }
}

// Per-lane byte offsets, within their 16-key group, of this lane's K and V
// transfers (issue_tile's rows and chunks) for a tile that lies wholly below
// nkeys, where no position is clamped: the same for every such tile.
template <int D>
struct DmaOffs {
  uint32_t k[8 / Geo<D>::kRowsPerLoad], v[8 / Geo<D>::kRowsPerLoad];
};
template <int D>
__device__ __forceinline__ DmaOffs<D> dma_offsets(int wave, int lane) {
  using Gm = Geo<D>;
  constexpr int RPL = Gm::kRowsPerLoad;
  const int sub = lane / Gm::kChunks, pc = lane % Gm::kChunks;
  DmaOffs<D> o;
#pragma unroll
  for (int j = 0; j < 8 / RPL; ++j) {
    const int R = 8 * wave + RPL * j + sub;
    const int kin = k_key_of_row(R) - 32 * (wave >> 2) - 16 * (wave & 1);  // key in its group
    o.k[j] = (uint32_t)((kin * D + (pc ^ k_swz<D>(R)) * 8) * 2);
    const int key = 8 * wave + RPL * j + sub;
    const int vin = key - 16 * (wave >> 1);
    o.v[j] = (uint32_t)((vin * D + (pc ^ v_swz<D>(key)) * 8) * 2);
  }
  return o;
}

// issue_tile for a tile with kbase + 64 <= nkeys, from the precomputed
// offsets: per transfer only the group's page base, which is uniform.
template <int D>
__device__ __forceinline__ void issue_tile_full(const Args &a, const long long *gtab, int g0, int kbase,
                                                const DmaOffs<D> &off, uint8_t *kdst, uint8_t *vdst,
                                                int wave) {
  using Gm = Geo<D>;
  constexpr int RPL = Gm::kRowsPerLoad;
  const uint16_t *kb = a.kpool + uniform_i64(gtab[kbase / 16 + 2 * (wave >> 2) + (wave & 1) - g0]);
  const uint16_t *vb = a.vpool + uniform_i64(gtab[kbase / 16 + (wave >> 1) - g0]);
#pragma unroll
  for (int j = 0; j < 8 / RPL; ++j)
    dma16_s(kb, off.k[j], (CFA_LDS void *)(kdst + (8 * wave + RPL * j) * Gm::kRowBytes));
#pragma unroll
  for (int j = 0; j < 8 / RPL; ++j)
    dma16_s(vb, off.v[j], (CFA_LDS void *)(vdst + (8 * wave + RPL * j) * Gm::kRowBytes));
}

// Visibility of the 64 keys kbase.. of a tile to a query whose ancestor mask
// (bits < N) is anc: context positions (< ctx) are all visible, tree position
// ctx + j is visible iff bit j of anc is set, positions past the tree never.
__device__ __forceinline__ uint64_t tile_visibility(int kbase, int ctx, uint64_t anc) {
  const int nctx = ctx - kbase;  // context keys at the start of the tile
  const uint64_t ctx_bits = nctx >= 64 ? ~0ull : (nctx <= 0 ? 0ull : ((1ull << nctx) - 1));
  // tile key k is tree node k - nctx
  const uint64_t tree_bits = nctx >= 0 ? (nctx >= 64 ? 0ull : anc << nctx)
                                       : (-nctx >= 64 ? 0ull : anc >> -nctx);
  return ctx_bits | tree_bits;
}

// Maximum over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four lanes holding
// one query column) without an LDS round trip: each permlane swap returns the
// lane's own value and its partner's (in one order or the other), so the max
// of the pair is the max of the two lanes.
__device__ __forceinline__ float column_max(float v) {
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}

// Per-wave state of the pipelined loop: 16-row query tiles qt of this wave,
// scores of one 64-key tile s[qt][blk][T] (keys blk*32 + 8g + 4T + i) and its
// bf16 probabilities p[qt][blk] (keys blk*32 + 8g + 0..7).
struct Scores {
  f32x4 s[kQT][2][2];
};
struct Probs {
  bf16x8 p[kQT][2];
};

template <int D>
struct Lane {
  bf16x8 qf[kQT][D / 32];  // Q^T columns pre-scaled by scale*log2(e)
  uint64_t anc[kQT];       // ancestor-or-self masks of the wave's columns
  int koff[D / 32];        // K-tile LDS byte offsets of this lane's operand reads
  int vbase, vh;           // V-tile transposed-read offset and swizzle
  int g;                   // lane / 16
};

// S^T = K Q^T - base: the accumulators start at -b so that the products come
// out relative to the column's exponent base.
template <int D>
__device__ __forceinline__ void qk_tile(const Lane<D> &ln, const uint8_t *Ks, const float *b,
                                        Scores &S) {
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int T = 0; T < 2; ++T) S.s[qt][blk][T] = f32x4{-b[qt], -b[qt], -b[qt], -b[qt]};
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        const uint4 kv = *reinterpret_cast<const uint4 *>(Ks + (blk * 32 + T * 16) * Geo<D>::kRowBytes +
                                                          ln.koff[kk]);
        const bf16x8 kf = __builtin_bit_cast(bf16x8, kv);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
          S.s[qt][blk][T] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, ln.qf[qt][kk], S.s[qt][blk][T], 0, 0, 0);
      }
}

// Online-softmax bookkeeping of one column: b is the exponent base (log2
// units) the scores are relative to, valid says b has been set.
struct Softmax {
  float b[kQT];
  bool valid[kQT];
};

// VALU phase of tile t: mask (tiles reaching the tree), column maxima, the
// rare rebase, and the probabilities P = exp2(S) in bf16.  S holds tile t's
// scores relative to each column's exponent base b; the base only moves when
// a column's maximum exceeds it by more than kRescaleSlack, which also
// rescales O and l (they hold tiles < t, so this precedes tile t's PV).
template <int D>
__device__ __forceinline__ void valu_phase(const Lane<D> &ln, int kbase, int ctx, Scores &S,
                                           Softmax &sm, f32x4 (&o)[kQT][D / 16],
                                           f32x4 (&lacc)[kQT], Probs &P) {
  if (kbase + kKT > ctx) {
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      // bit k: tile key k is visible to this column; this lane's keys are
      // blk*32 + 8g + 4T + i, i.e. bit blk*32 + 4T + i of vis >> 8g
      const uint64_t vis = tile_visibility(kbase, ctx, ln.anc[qt]) >> (8 * ln.g);
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            S.s[qt][blk][T][i] =
                ((vis >> (blk * 32 + 4 * T + i)) & 1ull) ? S.s[qt][blk][T][i] : -INFINITY;
    }
  }
  float mx[kQT];
  bool resc[kQT];
  bool any = false;
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    float v = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int i = 0; i < 4; ++i) v = fmaxf(v, S.s[qt][blk][T][i]);
    mx[qt] = column_max(v);
    resc[qt] = mx[qt] > -INFINITY && (!sm.valid[qt] || mx[qt] > kRescaleSlack);
    any |= resc[qt];
  }
  if (__ballot(any) != 0) {
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      const float d = resc[qt] ? mx[qt] : 0.0f;
      const float alpha = resc[qt] ? (sm.valid[qt] ? __builtin_amdgcn_exp2f(-d) : 0.0f) : 1.0f;
      sm.b[qt] += d;
      sm.valid[qt] = sm.valid[qt] || resc[qt];
      lacc[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) o[qt][dt] *= alpha;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int T = 0; T < 2; ++T) S.s[qt][blk][T] -= d;
    }
  }
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          P.p[qt][blk][T * 4 + i] = (__bf16)__builtin_amdgcn_exp2f(S.s[qt][blk][T][i]);
  // keep the exponentials in this phase: without a use here the compiler
  // sinks them past the phase barrier, next to the MFMAs that read them
  asm volatile("" ::"v"(P.p[0][0]), "v"(P.p[0][1]), "v"(P.p[1][0]), "v"(P.p[1][1]));
}

// MFMA phase of tile t: O^T += V_t^T P^T and l += 1^T P^T, then
// S = K_{t+1} Q^T - b (tile t+1's scores; for the last tile the stage read is
// stale and the result unused).  The QK products run k-slice outermost so
// that eight independent accumulation chains interleave: a dependent MFMA
// issued right behind its predecessor stalls the matrix pipe.  Lane (g, col)
// reads V rows blk*32 + 8g + 0..7 at d = dt*16 + col through two transposed
// 4x16 reads.
template <int D>
__device__ __forceinline__ void mfma_phase(const Lane<D> &ln, const uint8_t *Knext, const uint8_t *Vs,
                                           const float *b, const Probs &P, Scores &S,
                                           f32x4 (&o)[kQT][D / 16], f32x4 (&lacc)[kQT]) {
  constexpr int RB = Geo<D>::kRowBytes;
  bf16x8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = (__bf16)1.0f;
  f32x4 negb[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) negb[qt] = f32x4{-b[qt], -b[qt], -b[qt], -b[qt]};
  // the column sums first: they read no LDS, so they cover the latency of
  // the phase's first operand reads (about 1.5%)
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt)
      lacc[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, P.p[qt][blk], lacc[qt], 0, 0, 0);
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      const uint8_t *vp = Vs + blk * 32 * RB + ln.vbase + ((dt ^ ln.vh) << 5);
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((CFA_LDS i16x4 *)vp);
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((CFA_LDS i16x4 *)(vp + 4 * RB));
      const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt)
        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, P.p[qt][blk], o[qt][dt], 0, 0, 0);
    }
  }
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        const bf16x8 kf = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4 *>(Knext + (blk * 32 + T * 16) * RB + ln.koff[kk]));
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
          S.s[qt][blk][T] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              kf, ln.qf[qt][kk], kk == 0 ? negb[qt] : S.s[qt][blk][T], 0, 0, 0);
      }
#if CFA_TA_SGB
  // software pipeline of the operand reads: four fragments ahead, then two
  // reads after every pair of MFMAs
  __builtin_amdgcn_sched_group_barrier(0x0100, 8, 0);
#pragma unroll
  for (int j = 0; j < Geo<D>::kMfma / 2; ++j) {
    __builtin_amdgcn_sched_group_barrier(0x0008, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x0100, 2, 0);
  }
#endif
}

template <int D>
__global__ __launch_bounds__(kNT) void tree_attn_kernel(Args a) {
  using Gm = Geo<D>;
  constexpr int kTileBytes = Gm::kTileBytes;
  constexpr int kLoadsPerTile = Gm::kLoadsPerTile;
  __shared__ __align__(16) uint8_t kring[kKStages * kTileBytes];
  __shared__ __align__(16) uint8_t vring[kVStages * kTileBytes];
  __shared__ long long gtab[kMaxGroups];
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int col = lane & 15, g = lane >> 4;
  // positions past the block table are never read (ctx_lens beyond the
  // table's capacity are clamped rather than trusted)
  const int cap = a.max_blocks * a.bs;
  const int ctx = min(max(a.ctx[b], 0), max(cap - a.N, 0));
  const int nkeys = min(ctx + a.N, cap);
  const int ntiles = (nkeys + kKT - 1) / kKT;
  const int t0 = split * a.tiles_per_split;
  const int t1 = min(ntiles, t0 + a.tiles_per_split);
  const int g0 = t0 * (kKT / 16);

  // query rows of this wave: r = (node - q0) * G + head-in-group; Q^T is
  // scaled by scale*log2(e) once here so that scores come out in log2 units
  Lane<D> ln;
  ln.g = g;
  bool qvalid[kQT];
  {
    const uint64_t node_bits = a.N >= 64 ? ~0ull : ((1ull << a.N) - 1);
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      const int r = (wave * kQT + qt) * 16 + col;
      qvalid[qt] = r < a.rows;
      const int nl = qvalid[qt] ? r / a.G : 0, hg = r % a.G;
      ln.anc[qt] = qvalid[qt] ? a.mask[(long long)b * a.mask_sb + a.q0 + nl] & node_bits : 0ull;
      const uint16_t *qp =
          a.q + (((long long)b * a.Nq + nl) * a.Hq + (long long)h * a.G + hg) * D;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) {
        const uint4 v = qvalid[qt] ? ld_g16(qp + kk * 32 + g * 8) : make_uint4(0, 0, 0, 0);
        const bf16x8 raw = __builtin_bit_cast(bf16x8, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) ln.qf[qt][kk][j] = (__bf16)((float)raw[j] * a.scale_log2);
      }
    }
  }
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk)
    ln.koff[kk] = col * Gm::kRowBytes + (((kk * 4 + g) ^ k_swz<D>(col)) << 4);
  {
    const int vrow = 8 * g + (col >> 2);
    ln.vh = v_swz<D>(vrow) >> 1;
    ln.vbase = vrow * Gm::kRowBytes + ((col >> 1) & 1) * 16 + (col & 1) * 8;
  }

  // this wave's share of tile u: whole tiles from the fixed offsets, the
  // last tile of the keys (clamped positions) through issue_tile
  const DmaOffs<D> doff = dma_offsets<D>(wave, lane);
  auto issue = [&](int u, uint8_t *kdst, uint8_t *vdst) {
    if (u * kKT + kKT <= nkeys)
      issue_tile_full<D>(a, gtab, g0, u * kKT, doff, kdst, vdst, wave);
    else
      issue_tile<D>(a, gtab, g0, u * kKT, nkeys, kdst, vdst, wave, lane);
  };
  // the split's page lookups, once
  {
    const int32_t *btb = a.bt + (long long)b * a.max_blocks;
    const int ng = (t1 - t0) * (kKT / 16);
    for (int i = tid; i < ng; i += kNT) gtab[i] = group_row_offset<D>(a, btb, g0 + i, nkeys, h);
  }
  // Q and the table are in; settling every load here also tells the compiler
  // that nothing it issued is outstanding inside the loop below
  wait_vmcnt<0>();
  __syncthreads();

  f32x4 o[kQT][D / 16];
  f32x4 lacc[kQT];
  Softmax sm;
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    sm.b[qt] = 0.0f;
    sm.valid[qt] = false;
    lacc[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) o[qt][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  if (t0 < t1) {
    for (int u = t0; u < min(t0 + 3, t1); ++u)
      issue(u, kring + ((u - t0) % kKStages) * kTileBytes, vring + ((u - t0) % kVStages) * kTileBytes);
    // tile t0 has landed once at most the other prologue tiles are in flight
    const int later = min(t0 + 3, t1) - 1 - t0;
    if (later >= 2) wait_vmcnt<2 * kLoadsPerTile>();
    else if (later == 1) wait_vmcnt<kLoadsPerTile>();
    else wait_vmcnt<0>();
    block_barrier();
    // Waves w and w + 4 share a SIMD.  Group 1 (waves 4..7) runs one phase
    // behind group 0, so while one wave of a SIMD is in its VALU phase the
    // other is in its MFMA phase.  Barrier k ties group 0's phase k to group
    // 1's phase k - 1; group 1 takes one extra barrier first, group 0 one at
    // the end.  Tile t+1 must be visible before barrier 2(t - t0) + 1 (the
    // first MFMA phase reading it follows that barrier).  Tile t + 3 goes to
    // the stages of tiles t - 1 (K) and t - 2 (V), whose last readers (the
    // MFMA phases t - 2) finished before barrier 2(t - t0) - 1, so each group
    // issues its share before a VALU phase: group 0 after barrier 2(t - t0),
    // group 1 after barrier 2(t - t0) + 1.  No MFMA phase waits behind the
    // transfers' issue.
    const bool lag = wave >= kWaves / 2;
    if (lag) block_barrier();
    Scores S;
    Probs P;
    // a wave without query rows (few query nodes) only moves data and keeps
    // the barriers; its products would be discarded
    const bool busy = wave * kQT * 16 < a.rows;  // wave-uniform
    if (busy) qk_tile(ln, kring, sm.b, S);
    for (int t = t0; t < t1; ++t) {
      const int kbase = t * kKT;
      if (!lag) {
        block_barrier();
        if (t + 3 < t1) {
          const int u = t + 3 - t0;
          issue(t + 3, kring + (u % kKStages) * kTileBytes, vring + (u % kVStages) * kTileBytes);
        }
      } else {
        if (t + 2 < t1) wait_vmcnt<kLoadsPerTile>();
        else wait_vmcnt<0>();
        block_barrier();
        if (t + 3 < t1) {
          const int u = t + 3 - t0;
          issue(t + 3, kring + (u % kKStages) * kTileBytes, vring + (u % kVStages) * kTileBytes);
        }
      }
      if (busy) valu_phase(ln, kbase, ctx, S, sm, o, lacc, P);
      if (!lag) {
        if (t + 3 < t1) wait_vmcnt<2 * kLoadsPerTile>();
        else if (t + 2 < t1) wait_vmcnt<kLoadsPerTile>();
        else wait_vmcnt<0>();
        block_barrier();
      } else {
        block_barrier();
      }
      // the SIMD's other wave is in its VALU phase meanwhile: the MFMA
      // phase's issue goes first, its VALU work fills the MFMAs' shadow
      __builtin_amdgcn_s_setprio(1);
      if (busy)
        mfma_phase(ln, kring + ((t + 1 - t0) % kKStages) * kTileBytes,
                 vring + ((t - t0) % kVStages) * kTileBytes, sm.b, P, S, o, lacc);
      __builtin_amdgcn_s_setprio(0);
    }
    if (!lag) block_barrier();
  }

  // every lane holds its column's full sum; write final or partial outputs
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const float ls = lacc[qt][0];
    if (!qvalid[qt]) continue;
    const int r = (wave * kQT + qt) * 16 + col;
    if (a.splits == 1) {
      const int nl = r / a.G, hg = r % a.G;
      uint16_t *op = a.out + (((long long)b * a.Nq + nl) * a.Hq + (long long)h * a.G + hg) * D;
      const float inv = (ls > 0.0f) ? 1.0f / ls : 0.0f;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        uint16_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __builtin_bit_cast(uint16_t, (__bf16)(o[qt][dt][i] * inv));
        uint2 w;
        w.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
        w.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
        *reinterpret_cast<uint2 *>(op + dt * 16 + 4 * g) = w;
      }
    } else {
      // normalised partial in bf16 (the merge weighs it by its sum l)
      const long long prow = (((long long)split * a.B + b) * a.Hkv + h) * a.rows + r;
      uint16_t *pp = a.part_o + prow * D;
      const float inv = (ls > 0.0f) ? 1.0f / ls : 0.0f;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        uint2 w;
        w.x = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(o[qt][dt][0] * inv)) |
              ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(o[qt][dt][1] * inv)) << 16);
        w.y = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(o[qt][dt][2] * inv)) |
              ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(o[qt][dt][3] * inv)) << 16);
        *reinterpret_cast<uint2 *>(pp + dt * 16 + 4 * g) = w;
      }
      if (g == 0) a.part_ml[prow] = make_float2(sm.valid[qt] ? sm.b[qt] : -INFINITY, ls);
    }
  }
}

// Log-sum-exp merge of the splits: out = sum_s w_s l_s o_s / sum_s w_s l_s
// with w_s = 2^(m_s - max m) and o_s the normalised bf16 partial; D / 8
// threads per query row, eight d-values (one 16-byte load per split) per
// thread, 2048 / D rows per work-group.  Up to kMergeRegs splits are loaded in
// one round before any arithmetic.
constexpr int kMergeRegs = 4;  // splits merged from registers in one round of loads
template <int D>
__global__ __launch_bounds__(256) void tree_merge_kernel(Args a) {
  constexpr int kTPR = D / 8;  // threads per row
  const long long row_g = (long long)blockIdx.x * (256 / kTPR) + threadIdx.x / kTPR;
  const int q8 = threadIdx.x % kTPR;
  const long long total = (long long)a.B * a.Hkv * a.rows;
  if (row_g >= total) return;
  const int r = (int)(row_g % a.rows);
  const int h = (int)((row_g / a.rows) % a.Hkv);
  const int b = (int)(row_g / ((long long)a.rows * a.Hkv));
  const long long split_stride = (long long)a.B * a.Hkv * a.rows;  // rows per split
  const long long prow0 = ((long long)b * a.Hkv + h) * a.rows + r;
  float L = 0.0f;
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  auto add = [&](float w, const uint4 &v) {
    const uint32_t *vs = reinterpret_cast<const uint32_t *>(&v);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] += w * __uint_as_float(vs[j] << 16);
      acc[2 * j + 1] += w * __uint_as_float(vs[j] & 0xffff0000u);
    }
  };
  if (a.splits <= kMergeRegs) {
    // every split's (base, sum) and partial in flight at once
    float2 ml[kMergeRegs];
    uint4 v[kMergeRegs];
#pragma unroll
    for (int s = 0; s < kMergeRegs; ++s) {
      if (s < a.splits) {
        const long long prow = prow0 + s * split_stride;
        ml[s] = a.part_ml[prow];
        v[s] = *reinterpret_cast<const uint4 *>(a.part_o + prow * D + 8 * q8);
      }
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < kMergeRegs; ++s)
      if (s < a.splits) M = fmaxf(M, ml[s].x);
    const float base = (M == -INFINITY) ? 0.0f : M;
#pragma unroll
    for (int s = 0; s < kMergeRegs; ++s) {
      if (s < a.splits) {
        const float w = __builtin_amdgcn_exp2f(ml[s].x - base) * ml[s].y;
        L += w;
        add(w, v[s]);
      }
    }
  } else {
    float M = -INFINITY;
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, a.part_ml[prow0 + s * split_stride].x);
    const float base = (M == -INFINITY) ? 0.0f : M;
#pragma unroll 4
    for (int s = 0; s < a.splits; ++s) {
      const long long prow = prow0 + s * split_stride;
      const float2 ml = a.part_ml[prow];
      const uint4 v = *reinterpret_cast<const uint4 *>(a.part_o + prow * D + 8 * q8);
      const float w = __builtin_amdgcn_exp2f(ml.x - base) * ml.y;
      L += w;
      add(w, v);
    }
  }
  const float inv = (L > 0.0f) ? 1.0f / L : 0.0f;
  const int nl = r / a.G, hg = r % a.G;
  uint16_t *op = a.out + (((long long)b * a.Nq + nl) * a.Hq + (long long)h * a.G + hg) * D;
  uint4 w;
  uint32_t *ws = reinterpret_cast<uint32_t *>(&w);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    ws[j] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(acc[2 * j] * inv)) |
            ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(acc[2 * j + 1] * inv)) << 16);
  *reinterpret_cast<uint4 *>(op + 8 * q8) = w;
}

}  // namespace tree
}  // namespace cfa

using namespace cfa;
using namespace cfa::tree;

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

static void split_plan(int B, int Hkv, int max_keys, int splits_req, int &splits, int &tps) {
  const int tiles = std::max(1, (max_keys + kKT - 1) / kKT);
  int s = splits_req;
  if (s <= 0) {
    const int cus = abi::device_cu_count();
    const int items = std::max(1, B * Hkv);
    s = std::max(1, (cus + items - 1) / items);  // about one work-group per compute unit
  }
  // a split covers at most kMaxTilesPerSplit tiles (its page lookups fit LDS)
  s = std::max(s, (tiles + kMaxTilesPerSplit - 1) / kMaxTilesPerSplit);
  s = std::min(s, tiles);
  tps = (tiles + s - 1) / s;
  splits = (tiles + tps - 1) / tps;
}

extern "C" size_t cfa_tree_attention_workspace_size(int B, int N, int n_q_heads, int n_kv_heads,
                                                    int head_dim, int max_keys, int num_splits) {
  if (B <= 0 || N <= 0 || n_kv_heads <= 0 || n_q_heads <= 0 || (head_dim != 64 && head_dim != 128))
    return 0;
  int splits = 1, tps = 1;
  split_plan(B, n_kv_heads, max_keys, num_splits, splits, tps);
  if (splits == 1) return 256;
  const int G = n_q_heads / n_kv_heads;
  const size_t rows = (size_t)G * N;
  const size_t prows = (size_t)splits * B * n_kv_heads * rows;
  return align256(prows * head_dim * sizeof(uint16_t)) + align256(prows * sizeof(float2));
}

extern "C" int cfa_tree_attention(const void *q, const void *k_pool, const void *v_pool,
                                  const int32_t *block_tables, int max_blocks_per_seq,
                                  const int32_t *ctx_lens, int num_blocks, int num_layers,
                                  int layer, int block_size, const uint64_t *tree_mask,
                                  int64_t tree_mask_stride_b, int B, int N, int first_node,
                                  int n_q_heads,
                                  int n_kv_heads, int head_dim, float sm_scale, int max_keys,
                                  int num_splits, void *out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (!q || !k_pool || !v_pool || !block_tables || !ctx_lens || !tree_mask || !out)
    return fail_arg("null pointer argument");
  if (B <= 0 || N <= 0 || N > 64) return fail_arg("need B > 0 and 0 < N <= 64 tree nodes");
  if (first_node < 0 || first_node >= N) return fail_arg("need 0 <= first_node < N");
  if (head_dim != 64 && head_dim != 128) return fail_arg("head_dim must be 64 or 128");
  if (n_kv_heads <= 0 || n_q_heads <= 0 || n_q_heads % n_kv_heads)
    return fail_arg("n_q_heads must be a positive multiple of n_kv_heads");
  const int G = n_q_heads / n_kv_heads;
  const int Nq = N - first_node;
  if (G * Nq > kMaxRows)
    return fail_arg("(n_q_heads / n_kv_heads) * (N - first_node) must be at most 256");
  if (block_size <= 0 || block_size % 16) return fail_arg("block_size must be a multiple of 16");
  if (num_blocks <= 0 || num_layers <= 0 || layer < 0 || layer >= num_layers)
    return fail_arg("bad pool geometry (num_blocks, num_layers, layer)");
  if (max_keys < N) return fail_arg("max_keys must be at least N (context + tree tokens)");
  if ((long long)max_blocks_per_seq * block_size < max_keys)
    return fail_arg("max_blocks_per_seq * block_size must cover max_keys");
  if (B > 65535) return fail_arg("B must be at most 65535");
  Args a{};
  a.q = (const uint16_t *)q;
  a.kpool = (const uint16_t *)k_pool;
  a.vpool = (const uint16_t *)v_pool;
  a.bt = block_tables;
  a.ctx = ctx_lens;
  a.mask = tree_mask;
  a.mask_sb = tree_mask_stride_b;
  a.out = (uint16_t *)out;
  a.B = B;
  a.N = N;
  a.Hq = n_q_heads;
  a.Hkv = n_kv_heads;
  a.G = G;
  a.q0 = first_node;
  a.Nq = Nq;
  a.rows = G * Nq;
  a.max_blocks = max_blocks_per_seq;
  a.num_blocks = num_blocks;
  a.num_layers = num_layers;
  a.layer = layer;
  a.bs = block_size;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  split_plan(B, n_kv_heads, max_keys, num_splits, a.splits, a.tiles_per_split);
  const size_t need = cfa_tree_attention_workspace_size(B, Nq, n_q_heads, n_kv_heads, head_dim,
                                                        max_keys, num_splits);
  if (a.splits > 1) {
    if (!workspace || workspace_bytes < need)
      return fail_arg("workspace too small (see cfa_tree_attention_workspace_size)");
    const size_t prows = (size_t)a.splits * B * n_kv_heads * a.rows;
    a.part_o = (uint16_t *)workspace;
    a.part_ml = (float2 *)((char *)workspace + align256(prows * head_dim * sizeof(uint16_t)));
  }
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(a.splits, n_kv_heads, B);
  const long long rows = (long long)B * n_kv_heads * a.rows;
  if (head_dim == 128) {
    CFA_LAUNCH("tree_attn", tree_attn_kernel<128>, grid, dim3(kNT), 0, st, a);
    if (a.splits > 1)
      CFA_LAUNCH("tree_attn_merge", tree_merge_kernel<128>, dim3((unsigned)((rows + 15) / 16)),
                 dim3(256), 0, st, a);
  } else {
    CFA_LAUNCH("tree_attn", tree_attn_kernel<64>, grid, dim3(kNT), 0, st, a);
    if (a.splits > 1)
      CFA_LAUNCH("tree_attn_merge", tree_merge_kernel<64>, dim3((unsigned)((rows + 31) / 32)),
                 dim3(256), 0, st, a);
  }
  return CFA_OK;
}
