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
// rows (two 16-row tiles each) and share one LDS-staged 64-key K/V tile per
// step (double-buffered, register-prefetched).  Everything is computed in the
// transposed form
//   S^T = K Q^T            (MFMA A = K rows, B = Q^T columns)
//   O^T += V^T P^T         (MFMA A = V^T rows, B = P^T columns)
// so that each lane owns one query column throughout: the softmax of a column
// and the rescale of its O^T column stay in registers, and the P^T operand of
// the second product is the first product's output, converted to bf16 in
// place.  Within a 32-key block the two 16-key MFMA tiles take keys
// {8g+i} and {8g+4+i} (g = lane / 16, i < 4) so that lane (g, q) ends up with
// keys 8g..8g+7 of column q, which is exactly its 8-element k-slice of P^T.
// V is staged transposed in LDS so that the matching V^T k-slice is one
// 16-byte read.  Splits of the key range are merged by a log-sum-exp pass.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "abi_internal.hpp"

namespace cfa {
namespace tree {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;           // head_dim
constexpr int kKT = 64;           // keys per LDS tile
constexpr int kWaves = 8;
constexpr int kNT = kWaves * 64;  // threads per work-group
constexpr int kQT = 2;            // 16-row query tiles per wave
constexpr int kMaxRows = kWaves * kQT * 16;  // 256 query rows per work-group
constexpr int kKPad = kD + 8;     // K row stride in LDS (bf16), breaks bank aliasing
constexpr int kVPad = kKT + 8;    // V^T row stride in LDS (bf16)

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
  float2 *part_ml;         // [S, B, Hkv, rows] (running max in log2 units, sum)
  int B, N, Hq, Hkv, G, rows;
  int max_blocks, num_blocks, num_layers, layer, bs;
  int splits, tiles_per_split;
  float scale_log2;        // sm_scale * log2(e)
};

struct __align__(16) Smem {
  uint16_t k[2][kKT * kKPad];
  uint16_t vt[2][kD * kVPad];
};

__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t *p) {
  const uint4 v = *reinterpret_cast<const uint4 *>(p);
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ uint4 ld_g16(const uint16_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}

// LDS row of key k within a tile: the two 16-key MFMA tiles of a 32-key
// block read keys {8g+i} and {8g+4+i}; storing key 8g + 4T + i at row
// 16T + 4g + i makes each MFMA tile read 16 consecutive rows, which a 272-byte
// row stride spreads over all 64 banks.
__device__ __forceinline__ int k_row(int key) {
  return (key & ~31) + ((key >> 2) & 1) * 16 + ((key >> 3) & 3) * 4 + (key & 3);
}

// Global staging of one 64-key tile.  K: thread t owns the 16-byte chunks
// (key t/16, slice t%16) and (key t/16 + 32, same slice).  V: lane l of wave
// w owns keys 2(l%32), 2(l%32)+1 at d-slice 2w + l/32, so that the transposed
// 4-byte LDS writes of one wave hit 64 distinct banks.
struct Stage {
  uint4 k0, k1;
  uint4 v0, v1;
};

// Element offsets (within a pool) of the tile's pages, read with uniform
// addresses: page j of the tile covers keys [j*bs, (j+1)*bs), j < kKT / bs.
struct Pages {
  long long o0, o1, o2, o3;
};

__device__ __forceinline__ long long page_off(const Args &a, const int32_t *btb, int page, int h) {
  page = min(page, a.max_blocks - 1);
  int blk = btb[page];
  blk = min(max(blk, 0), a.num_blocks - 1);  // stay inside the pool whatever the table holds
  return (((long long)blk * a.num_layers + a.layer) * a.Hkv + h) * (long long)(a.bs * kD);
}

__device__ __forceinline__ Pages tile_pages(const Args &a, int b, int h, int kbase) {
  const int32_t *btb = a.bt + (long long)b * a.max_blocks;
  const int p0 = kbase / a.bs, last = kKT / a.bs - 1;
  Pages pg;
  pg.o0 = page_off(a, btb, p0, h);
  pg.o1 = page_off(a, btb, p0 + min(1, last), h);
  pg.o2 = page_off(a, btb, p0 + min(2, last), h);
  pg.o3 = page_off(a, btb, p0 + min(3, last), h);
  return pg;
}

// Offset of the row of tile-relative key `key`.
__device__ __forceinline__ long long key_off(const Pages &pg, int bs, int key) {
  const int j = key / bs;
  long long o = pg.o0;
  o = (j == 1) ? pg.o1 : o;
  o = (j == 2) ? pg.o2 : o;
  o = (j == 3) ? pg.o3 : o;
  return o + (long long)((key % bs) * kD);
}

__device__ __forceinline__ void stage_load(const Args &a, int b, int h, int kbase, int nkeys,
                                           Stage &st) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint4 z = make_uint4(0, 0, 0, 0);
  const Pages pg = tile_pages(a, b, h, kbase);
  {
    const int key = tid >> 4, ds = tid & 15;
    st.k0 = (kbase + key < nkeys) ? ld_g16(a.kpool + key_off(pg, a.bs, key) + ds * 8) : z;
    st.k1 = (kbase + key + 32 < nkeys) ? ld_g16(a.kpool + key_off(pg, a.bs, key + 32) + ds * 8) : z;
  }
  {
    const int kp = lane & 31, ds = wave * 2 + (lane >> 5);
    const int key = 2 * kp;
    st.v0 = (kbase + key < nkeys) ? ld_g16(a.vpool + key_off(pg, a.bs, key) + ds * 8) : z;
    st.v1 = (kbase + key + 1 < nkeys) ? ld_g16(a.vpool + key_off(pg, a.bs, key + 1) + ds * 8) : z;
  }
}

__device__ __forceinline__ void stage_store(Smem &sm, int buf, const Stage &st) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  {
    const int key = tid >> 4, ds = tid & 15;
    *reinterpret_cast<uint4 *>(&sm.k[buf][k_row(key) * kKPad + ds * 8]) = st.k0;
    *reinterpret_cast<uint4 *>(&sm.k[buf][k_row(key + 32) * kKPad + ds * 8]) = st.k1;
  }
  {
    const int kp = lane & 31, ds = wave * 2 + (lane >> 5);
    const uint32_t a[4] = {st.v0.x, st.v0.y, st.v0.z, st.v0.w};
    const uint32_t c[4] = {st.v1.x, st.v1.y, st.v1.z, st.v1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // d = ds*8 + 2j (low halves) and + 1 (high halves); keys 2kp, 2kp+1
      const uint32_t lo = (a[j] & 0xffffu) | (c[j] << 16);
      const uint32_t hi = (a[j] >> 16) | (c[j] & 0xffff0000u);
      *reinterpret_cast<uint32_t *>(&sm.vt[buf][(ds * 8 + 2 * j) * kVPad + 2 * kp]) = lo;
      *reinterpret_cast<uint32_t *>(&sm.vt[buf][(ds * 8 + 2 * j + 1) * kVPad + 2 * kp]) = hi;
    }
  }
}

__device__ __forceinline__ float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m, 64)); }
__device__ __forceinline__ float xor_sum(float v, int m) { return v + __shfl_xor(v, m, 64); }

__global__ __launch_bounds__(kNT) void tree_attn_kernel(Args a) {
  __shared__ Smem sm;
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, g = lane >> 4;
  // positions past the block table are never read (ctx_lens beyond the
  // table's capacity are clamped rather than trusted)
  const int cap = a.max_blocks * a.bs;
  const int ctx = min(max(a.ctx[b], 0), max(cap - a.N, 0));
  const int nkeys = min(ctx + a.N, cap);
  const int ntiles = (nkeys + kKT - 1) / kKT;
  const int t0 = split * a.tiles_per_split;
  const int t1 = min(ntiles, t0 + a.tiles_per_split);

  // query rows of this wave: r = node * G + head-in-group
  bf16x8 qf[kQT][4];
  uint64_t anc[kQT];
  bool qvalid[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const int r = (wave * kQT + qt) * 16 + col;
    qvalid[qt] = r < a.rows;
    const int node = qvalid[qt] ? r / a.G : 0, hg = r % a.G;
    anc[qt] = qvalid[qt] ? a.mask[(long long)b * a.mask_sb + node] : 0ull;
    const uint16_t *qp = a.q + (((long long)b * a.N + node) * a.Hq + (long long)h * a.G + hg) * kD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint4 v = qvalid[qt] ? ld_g16(qp + kk * 32 + g * 8) : make_uint4(0, 0, 0, 0);
      qf[qt][kk] = __builtin_bit_cast(bf16x8, v);
    }
  }

  f32x4 o[kQT][kD / 16];
  float m[kQT], l[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < kD / 16; ++dt) o[qt][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  Stage st;
  if (t0 < t1) stage_load(a, b, h, t0 * kKT, nkeys, st);
  for (int t = t0; t < t1; ++t) {
    const int buf = (t - t0) & 1;
    stage_store(sm, buf, st);
    __syncthreads();
    if (t + 1 < t1) stage_load(a, b, h, (t + 1) * kKT, nkeys, st);
    const uint16_t *K = sm.k[buf];
    const uint16_t *Vt = sm.vt[buf];
    const int kbase = t * kKT;

    // S^T for the tile: s[qt][blk][T] holds keys blk*32 + T*4 + 8g + i
    f32x4 s[kQT][2][2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) s[qt][blk][T] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const int krow = blk * 32 + T * 16 + col;  // = k_row(blk*32 + T*4 + 8*(col/4) + col%4)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 kf = ld_bf16x8(K + krow * kKPad + kk * 32 + g * 8);
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt)
            s[qt][blk][T] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[qt][kk], s[qt][blk][T], 0, 0, 0);
        }
      }

    // mask, online softmax in log2 units (per query column; the 4 lanes g of
    // a column share it)
    const bool masked_tile = kbase + kKT > ctx;
    const float c = a.scale_log2;
    bf16x8 p[kQT][2];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      float tmax = -INFINITY;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = s[qt][blk][T][i];
            if (masked_tile) {
              const int pos = kbase + blk * 32 + T * 4 + 8 * g + i;
              const int j = pos - ctx;
              const bool vis = pos < ctx || (j < a.N && ((anc[qt] >> (j & 63)) & 1ull));
              v = vis ? v : -INFINITY;
            }
            s[qt][blk][T][i] = v;
            tmax = fmaxf(tmax, v);
          }
      tmax = xor_max(tmax, 16);
      tmax = xor_max(tmax, 32);
      const float mnew = fmaxf(m[qt], tmax * c);  // c > 0: max of scaled = scaled max
      const float base = (mnew == -INFINITY) ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(m[qt] - base);
      m[qt] = mnew;
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
      l[qt] = l[qt] * alpha + psum;
      if (alpha != 1.0f) {
#pragma unroll
        for (int dt = 0; dt < kD / 16; ++dt) o[qt][dt] *= alpha;
      }
    }

    // O^T += V^T P^T
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int dt = 0; dt < kD / 16; ++dt) {
        const bf16x8 vf = ld_bf16x8(Vt + (dt * 16 + col) * kVPad + blk * 32 + 8 * g);
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
  if (block_size <= 0 || kKT % block_size) return fail_arg("block_size must divide 64");
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
