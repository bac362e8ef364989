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
// been appended at positions ctx_b .. ctx_b + N - 1.
//
// One work-group = (split, kv head, sequence); its 8 waves hold all G*N query
// rows (two 16-row tiles each, Q^T in registers) and share a ring of
// kStages LDS stages, each holding one 64-key K tile and one 64-key V tile.
// Tiles move HBM -> LDS with direct 16-byte global_load_lds transfers (no
// register staging), kStages - 1 tiles ahead of the tile being computed.
// Everything is computed in the transposed form
//   S^T = K Q^T            (MFMA A = K rows, B = Q^T columns)
//   O^T += V^T P^T         (MFMA A = V^T rows, B = P^T columns)
// so each lane owns one query column throughout: the softmax of a column and
// the rescale of its O^T column stay in registers, and the P^T operand of the
// second product is the first product's output converted to bf16 in place.
// Within a 32-key block the two 16-key MFMA tiles take keys {8g+i} and
// {8g+4+i} (g = lane / 16, i < 4), so lane (g, q) ends up with keys 8g..8g+7
// of column q: exactly its 8-element k-slice of P^T.  The matching V^T
// k-slice comes from two ds_read_b64_tr_b16 transposed reads of the V tile,
// which stays in its natural [key][d] layout.
//
// LDS layouts (256-byte rows, 16-byte chunks XOR-swizzled so that the MFMA
// operand reads of one wave hit distinct banks):
//   K: row R holds key 32*(R/32) + 8*((R/4)%4) + 4*((R/16)%2) + R%4 (each
//      16-row MFMA tile reads consecutive rows); chunk c sits at c ^ (R % 16).
//   V: row = key; chunk c sits at c ^ 2*((key % 4) | 4*((key / 8) % 2)).
//
// Softmax rescaling is lazy: a column's exponent base only moves when its
// running maximum grows by more than kRescaleSlack (log2 units), so P^T
// entries stay below 2^kRescaleSlack and the O^T rescale is rare.  Splits of
// the key range are merged by a log-sum-exp pass.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "abi_internal.hpp"

#define CFA_LDS __attribute__((address_space(3)))

namespace cfa {
namespace tree {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;                       // head_dim
constexpr int kKT = 64;                       // keys per tile
constexpr int kWaves = 8;
constexpr int kNT = kWaves * 64;              // threads per work-group
constexpr int kQT = 2;                        // 16-row query tiles per wave
constexpr int kMaxRows = kWaves * kQT * 16;   // 256 query rows per work-group
constexpr int kRowBytes = kD * 2;             // one K or V row, bf16
constexpr int kTileBytes = kKT * kRowBytes;   // 16 KiB
constexpr int kStages = 3;                    // LDS ring depth (tiles)
constexpr int kStageBytes = 2 * kTileBytes;   // K tile then V tile
constexpr int kLoadsPerTile = 4;              // global_load_lds per wave per tile
constexpr float kRescaleSlack = 8.0f;         // log2 units
constexpr int kMaxGroups = 1024;              // 16-key groups per split (page lookup table)
constexpr int kMaxTilesPerSplit = kMaxGroups / (kKT / 16);

struct Args {
  const uint16_t *q;       // [B, N, Hq, D]
  const uint16_t *kpool;   // [blocks, layers, Hkv, bs, D]
  const uint16_t *vpool;
  const int32_t *bt;       // [B, max_blocks]
  const int32_t *ctx;      // [B]
  const uint64_t *mask;    // [N] or [B, N]
  long long mask_sb;
  uint16_t *out;           // [B, N, Hq, D]
  float *part_o;           // [S, B, Hkv, rows, D] unnormalised partial outputs
  float2 *part_ml;         // [S, B, Hkv, rows] (exponent base in log2 units, sum)
  int B, N, Hq, Hkv, G, rows;
  int max_blocks, num_blocks, num_layers, layer, bs;
  int splits, tiles_per_split;
  float scale_log2;        // sm_scale * log2(e)
};

__device__ __forceinline__ uint4 ld_g16(const uint16_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}

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

// Work-group barrier without the release/acquire fences of __syncthreads
// (those would wait for every outstanding transfer); the empty asm statements
// keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Key (tile-relative) held by K-tile LDS row R.
__device__ __forceinline__ int k_key_of_row(int R) {
  return (R & ~31) + ((R >> 2) & 3) * 8 + ((R >> 4) & 1) * 4 + (R & 3);
}

// Swizzle of V-tile row `key`: 2 * ((key % 4) | 4 * ((key / 8) % 2)).
__device__ __forceinline__ int v_swz(int key) { return ((key & 3) | ((key >> 1) & 4)) << 1; }

// Pool element offset of the row holding position gstart = min(16 gi,
// nkeys - 1), the first row 16-key group gi reads.  Page index and block id
// are clamped into the table and the pool, so a corrupt table can never send
// a load outside the pool.
__device__ __forceinline__ long long group_row_offset(const Args &a, const int32_t *btb, int gi,
                                                      int nkeys, int h) {
  const int gstart = min(gi * 16, nkeys - 1);
  const int page = min(gstart / a.bs, a.max_blocks - 1);
  const int blk = min(max(btb[page], 0), a.num_blocks - 1);
  return (((long long)blk * a.num_layers + a.layer) * a.Hkv + h) * (long long)(a.bs * kD) +
         (long long)(gstart - page * a.bs) * kD;
}

__device__ __forceinline__ long long uniform_i64(long long v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((unsigned long long)v >> 32));
  return (long long)(((unsigned long long)hi << 32) | lo);
}

// Issue this wave's share of the tile at key kbase: two 1 KiB K transfers
// (LDS rows 8w..8w+7) and two 1 KiB V transfers (keys 8w..8w+7).  Each
// transfer covers four keys of one 16-key group, and a group never straddles
// a page (block_size % 16 == 0).  Keys at or past nkeys re-read key
// nkeys - 1: a finite, in-bounds row that the mask then hides.  gtab holds
// the split's group row offsets (group_row_offset) from group g0 on.
__device__ __forceinline__ void issue_tile(const Args &a, const long long *gtab, int g0, int kbase,
                                           int nkeys, uint8_t *stage, int wave, int lane) {
  const int sub = lane >> 4, pc = lane & 15;
  {
    // K: the wave's rows hold keys of the tile's 16-group 2 (w / 4) + (w % 2)
    const int gi = kbase / 16 + 2 * (wave >> 2) + (wave & 1);
    const int gstart = min(gi * 16, nkeys - 1);
    const uint16_t *base = a.kpool + uniform_i64(gtab[gi - g0]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int R = 8 * wave + 4 * j + sub;
      const int c = pc ^ (R & 15);
      const int pos = min(kbase + k_key_of_row(R), nkeys - 1);
      dma16(base + ((pos - gstart) * kD + c * 8),
            (CFA_LDS void *)(stage + (8 * wave + 4 * j) * kRowBytes));
    }
  }
  {
    // V: keys 8w..8w+7, in the tile's 16-group w / 2
    const int gi = kbase / 16 + (wave >> 1);
    const int gstart = min(gi * 16, nkeys - 1);
    const uint16_t *base = a.vpool + uniform_i64(gtab[gi - g0]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int key = 8 * wave + 4 * j + sub;
      const int c = pc ^ v_swz(key);
      const int pos = min(kbase + key, nkeys - 1);
      dma16(base + ((pos - gstart) * kD + c * 8),
            (CFA_LDS void *)(stage + kTileBytes + (8 * wave + 4 * j) * kRowBytes));
    }
  }
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

__device__ __forceinline__ float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m, 64)); }
__device__ __forceinline__ float xor_sum(float v, int m) { return v + __shfl_xor(v, m, 64); }

__global__ __launch_bounds__(kNT) void tree_attn_kernel(Args a) {
  __shared__ __align__(16) uint8_t smem[kStages * kStageBytes];
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

  // query rows of this wave: r = node * G + head-in-group
  const uint64_t node_bits = a.N >= 64 ? ~0ull : ((1ull << a.N) - 1);
  bf16x8 qf[kQT][4];
  uint64_t anc[kQT];
  bool qvalid[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const int r = (wave * kQT + qt) * 16 + col;
    qvalid[qt] = r < a.rows;
    const int node = qvalid[qt] ? r / a.G : 0, hg = r % a.G;
    anc[qt] = qvalid[qt] ? a.mask[(long long)b * a.mask_sb + node] & node_bits : 0ull;
    const uint16_t *qp = a.q + (((long long)b * a.N + node) * a.Hq + (long long)h * a.G + hg) * kD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint4 v = qvalid[qt] ? ld_g16(qp + kk * 32 + g * 8) : make_uint4(0, 0, 0, 0);
      qf[qt][kk] = __builtin_bit_cast(bf16x8, v);
    }
  }

  // the split's page lookups, once
  {
    const int32_t *btb = a.bt + (long long)b * a.max_blocks;
    const int ng = (t1 - t0) * (kKT / 16);
    for (int i = tid; i < ng; i += kNT) gtab[i] = group_row_offset(a, btb, g0 + i, nkeys, h);
  }
  // Q and the table are in; settling every load here also tells the compiler
  // that nothing it issued is outstanding inside the loop below
  wait_vmcnt<0>();
  __syncthreads();

  // prologue: the first kStages - 1 tiles go in flight
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s)
    if (t0 + s < t1)
      issue_tile(a, gtab, g0, (t0 + s) * kKT, nkeys, smem + s * kStageBytes, wave, lane);

  f32x4 o[kQT][kD / 16];
  float m[kQT], l[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < kD / 16; ++dt) o[qt][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // per-lane LDS byte offsets, tile-relative
  int koff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) koff[kk] = col * kRowBytes + (((kk * 4 + g) ^ col) << 4);
  const int vrow = 8 * g + (col >> 2);
  const int vh = v_swz(vrow) >> 1;
  const int vbase = vrow * kRowBytes + ((col >> 1) & 1) * 16 + (col & 1) * 8;

  const float c = a.scale_log2;
  for (int t = t0; t < t1; ++t) {
    // this wave's transfers of tile t have landed once at most the later
    // tiles' transfers are outstanding; the barrier then publishes every
    // wave's transfers and retires the stage read during tile t - 1
    const int later = min(kStages - 2, t1 - 1 - t);
    if (later >= 1) wait_vmcnt<kLoadsPerTile * (kStages - 2)>();
    else wait_vmcnt<0>();
    block_barrier();
    if (t + kStages - 1 < t1)
      issue_tile(a, gtab, g0, (t + kStages - 1) * kKT, nkeys,
                 smem + ((t - t0 + kStages - 1) % kStages) * kStageBytes, wave, lane);
    const uint8_t *Ks = smem + ((t - t0) % kStages) * kStageBytes;
    const uint8_t *Vs = Ks + kTileBytes;
    const int kbase = t * kKT;

    // S^T for the tile: s[qt][blk][T] holds keys blk*32 + T*4 + 8g + i
    f32x4 s[kQT][2][2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) s[qt][blk][T] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const uint4 kv =
              *reinterpret_cast<const uint4 *>(Ks + (blk * 32 + T * 16) * kRowBytes + koff[kk]);
          const bf16x8 kf = __builtin_bit_cast(bf16x8, kv);
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt)
            s[qt][blk][T] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[qt][kk], s[qt][blk][T], 0, 0, 0);
        }
      }

    // mask (tiles reaching the tree only), then online softmax in log2 units
    // (per query column; the 4 lanes g of a column share it)
    if (kbase + kKT > ctx) {
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        // bit k: tile key k is visible to this column; this lane's keys are
        // blk*32 + 8g + 4T + i, i.e. bit blk*32 + 4T + i of vis >> 8g
        const uint64_t vis = tile_visibility(kbase, ctx, anc[qt]) >> (8 * g);
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int T = 0; T < 2; ++T)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              s[qt][blk][T][i] = ((vis >> (blk * 32 + 4 * T + i)) & 1ull) ? s[qt][blk][T][i] : -INFINITY;
      }
    }
    bf16x8 p[kQT][2];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      float tmax = -INFINITY;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[qt][blk][T][i]);
      tmax = xor_max(tmax, 16);
      tmax = xor_max(tmax, 32);
      const float mx = tmax * c;  // c > 0: max of scaled = scaled max
      if (mx > m[qt] + kRescaleSlack) {
        const float alpha = __builtin_amdgcn_exp2f(m[qt] - mx);  // 0 on the first visible tile
        m[qt] = mx;
        l[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < kD / 16; ++dt) o[qt][dt] *= alpha;
      }
      // m is -inf only while every key so far was masked (then so is this tile)
      const float base = (m[qt] == -INFINITY) ? 0.0f : m[qt];
      float psum = 0.0f;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        float pv[8];
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][blk][T][i], c, -base));
            pv[T * 4 + i] = e;
            psum += e;
          }
#pragma unroll
        for (int j = 0; j < 8; ++j) p[qt][blk][j] = (__bf16)pv[j];
      }
      l[qt] += psum;
    }

    // O^T += V^T P^T; lane (g, col) reads V rows blk*32 + 8g + 0..7 at
    // d = dt*16 + col through two transposed 4x16 reads
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int dt = 0; dt < kD / 16; ++dt) {
        const uint8_t *vp = Vs + blk * 32 * kRowBytes + vbase + ((dt ^ vh) << 5);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((CFA_LDS i16x4 *)vp);
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((CFA_LDS i16x4 *)(vp + 4 * kRowBytes));
        const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
          o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, p[qt][blk], o[qt][dt], 0, 0, 0);
      }
  }

  // column sums over the 4 lanes of a query; write final or partial outputs
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    float ls = xor_sum(l[qt], 16);
    ls = xor_sum(ls, 32);
    if (!qvalid[qt]) continue;
    const int r = (wave * kQT + qt) * 16 + col;
    if (a.splits == 1) {
      const int node = r / a.G, hg = r % a.G;
      uint16_t *op = a.out + (((long long)b * a.N + node) * a.Hq + (long long)h * a.G + hg) * kD;
      const float inv = (ls > 0.0f) ? 1.0f / ls : 0.0f;
#pragma unroll
      for (int dt = 0; dt < kD / 16; ++dt) {
        uint16_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __builtin_bit_cast(uint16_t, (__bf16)(o[qt][dt][i] * inv));
        uint2 w;
        w.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
        w.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
        *reinterpret_cast<uint2 *>(op + dt * 16 + 4 * g) = w;
      }
    } else {
      const long long prow = (((long long)split * a.B + b) * a.Hkv + h) * a.rows + r;
      float *pp = a.part_o + prow * kD;
#pragma unroll
      for (int dt = 0; dt < kD / 16; ++dt)
        *reinterpret_cast<f32x4 *>(pp + dt * 16 + 4 * g) = o[qt][dt];
      if (g == 0) a.part_ml[prow] = make_float2(m[qt], ls);
    }
  }
}

// Log-sum-exp merge of the splits: one wave per query row, 2 d-values per lane.
__global__ __launch_bounds__(256) void tree_merge_kernel(Args a) {
  const int row_g = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const long long total = (long long)a.B * a.Hkv * a.rows;
  if (row_g >= total) return;
  const int r = row_g % a.rows;
  const int h = (row_g / a.rows) % a.Hkv;
  const int b = row_g / (a.rows * a.Hkv);
  float M = -INFINITY;
  for (int s = 0; s < a.splits; ++s) {
    const long long prow = (((long long)s * a.B + b) * a.Hkv + h) * a.rows + r;
    M = fmaxf(M, a.part_ml[prow].x);
  }
  const float base = (M == -INFINITY) ? 0.0f : M;
  float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (int s = 0; s < a.splits; ++s) {
    const long long prow = (((long long)s * a.B + b) * a.Hkv + h) * a.rows + r;
    const float2 ml = a.part_ml[prow];
    const float w = __builtin_amdgcn_exp2f(ml.x - base);
    L += ml.y * w;
    const float2 ov = *reinterpret_cast<const float2 *>(a.part_o + prow * kD + 2 * lane);
    o0 += ov.x * w;
    o1 += ov.y * w;
  }
  const float inv = (L > 0.0f) ? 1.0f / L : 0.0f;
  const int node = r / a.G, hg = r % a.G;
  uint16_t *op = a.out + (((long long)b * a.N + node) * a.Hq + (long long)h * a.G + hg) * kD;
  const uint32_t w = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(o0 * inv)) |
                     ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(o1 * inv)) << 16);
  *reinterpret_cast<uint32_t *>(op + 2 * lane) = w;
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
  if (B <= 0 || N <= 0 || n_kv_heads <= 0 || n_q_heads <= 0 || head_dim != kD) return 0;
  int splits = 1, tps = 1;
  split_plan(B, n_kv_heads, max_keys, num_splits, splits, tps);
  if (splits == 1) return 256;
  const int G = n_q_heads / n_kv_heads;
  const size_t rows = (size_t)G * N;
  const size_t prows = (size_t)splits * B * n_kv_heads * rows;
  return align256(prows * kD * sizeof(float)) + align256(prows * sizeof(float2));
}

extern "C" int cfa_tree_attention(const void *q, const void *k_pool, const void *v_pool,
                                  const int32_t *block_tables, int max_blocks_per_seq,
                                  const int32_t *ctx_lens, int num_blocks, int num_layers,
                                  int layer, int block_size, const uint64_t *tree_mask,
                                  int64_t tree_mask_stride_b, int B, int N, int n_q_heads,
                                  int n_kv_heads, int head_dim, float sm_scale, int max_keys,
                                  int num_splits, void *out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (!q || !k_pool || !v_pool || !block_tables || !ctx_lens || !tree_mask || !out)
    return fail_arg("null pointer argument");
  if (B <= 0 || N <= 0 || N > 64) return fail_arg("need B > 0 and 0 < N <= 64 tree nodes");
  if (head_dim != kD) return fail_arg("head_dim must be 128");
  if (n_kv_heads <= 0 || n_q_heads <= 0 || n_q_heads % n_kv_heads)
    return fail_arg("n_q_heads must be a positive multiple of n_kv_heads");
  const int G = n_q_heads / n_kv_heads;
  if (G * N > kMaxRows) return fail_arg("(n_q_heads / n_kv_heads) * N must be at most 256");
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
  a.rows = G * N;
  a.max_blocks = max_blocks_per_seq;
  a.num_blocks = num_blocks;
  a.num_layers = num_layers;
  a.layer = layer;
  a.bs = block_size;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  split_plan(B, n_kv_heads, max_keys, num_splits, a.splits, a.tiles_per_split);
  const size_t need = cfa_tree_attention_workspace_size(B, N, n_q_heads, n_kv_heads, head_dim,
                                                        max_keys, num_splits);
  if (a.splits > 1) {
    if (!workspace || workspace_bytes < need)
      return fail_arg("workspace too small (see cfa_tree_attention_workspace_size)");
    const size_t prows = (size_t)a.splits * B * n_kv_heads * a.rows;
    a.part_o = (float *)workspace;
    a.part_ml = (float2 *)((char *)workspace + align256(prows * kD * sizeof(float)));
  }
  hipStream_t st = (hipStream_t)stream;
  CFA_LAUNCH("tree_attn", tree_attn_kernel, dim3(a.splits, n_kv_heads, B), dim3(kNT), 0, st, a);
  if (a.splits > 1) {
    const long long rows = (long long)B * n_kv_heads * a.rows;
    CFA_LAUNCH("tree_attn_merge", tree_merge_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
               st, a);
  }
  return CFA_OK;
}
