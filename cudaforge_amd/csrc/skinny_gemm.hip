// skinny_gemm.hip -- bf16 GEMM for few rows, C [M, N] = A [M, K] x W [K, N]
// with M <= 128 and W row-major (the layout of `x @ w`): the draft model's
// per-level projections, where the work is streaming W once.
//
// A work-group owns a 64-column tile of C and one of S equal k ranges
// (split-K).  Each pipeline step moves 128 rows of the W tile (16 KiB) and
// the matching 128-column slab of A by direct HBM -> LDS transfers into a
// ring (4 stages, 3 for M > 16), and wave w multiplies k-slice 32w .. 32w+31
// of the step on v_mfma_f32_16x16x32_bf16: the four waves cover disjoint k,
// so no byte of A or W is read twice from LDS.  W keeps its natural [k][n]
// layout; the B operand (8 consecutive k of one column per lane) comes from
// two ds_read_b64_tr_b16 transposed reads.  At the end the four waves'
// accumulators are summed through LDS in wave order; with S > 1 each
// work-group stores its fp32 partial tile, and the last of the S to arrive
// (an arrival counter per tile, reset by that work-group) sums the partials
// in split order.  Every sum has a fixed order, so results do not depend on
// scheduling.
//
// LDS layouts (16-byte chunks XOR-swizzled so that each operand read of a
// wave touches every bank once per 16 lanes):
//   W stage: row k (128 bytes, 64 columns), chunk c at position
//     c ^ w_swz(k), w_swz(k) = 2 (((k / 2) % 2) | 2 ((k / 8) % 2)).
//   A stage: row m (256 bytes, 128 k), chunk c at position c ^ (m % 16).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "abi_internal.hpp"
#include "lds_dma.hpp"
#include "silu.hpp"

namespace cfa {
namespace sg {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kNT = 64;                 // columns per work-group tile
constexpr int kKS = 128;                // k rows per pipeline step (32 per wave)
constexpr int kWBytes = kKS * kNT * 2;  // W part of a stage: 16 KiB
constexpr int kMaxM = 128;

struct Args {
  const uint16_t *A;  // [M, K]
  const uint16_t *W;  // [K, N]
  uint16_t *C;        // [M, N]; with the SiLU epilogue [M, N / 2]
  float *part;        // [tiles][S][4 MT blocks][4 elements][64 lanes]
  int *cnt;           // [tiles] arrival counters, zero between calls
  int M, N, K, S, tiles, steps;  // steps: pipeline steps per split
};

template <int MT>
struct Cfg {
  static constexpr int kABytes = MT * 16 * kKS * 2;
  static constexpr int kStage = kWBytes + kABytes;
  static constexpr int kStages = MT == 1 ? 4 : 3;
  static constexpr int kLds = kStages * kStage;
  static constexpr int kLPI = 4 + MT;  // transfers per wave per stage
  static_assert(kLds >= 4 * 4 * MT * 1024 + 4, "reduction area and flag exceed the ring");
  static_assert(kLds <= 160 * 1024, "LDS");
};

__device__ __forceinline__ int w_swz(int k) { return (((k >> 1) & 1) | ((k >> 2) & 2)) << 1; }

// s_waitcnt vmcnt(N) lgkmcnt(0): this wave's transfers of the stage have
// landed and its LDS reads of the previous stage have returned, so the
// barrier after it also frees the slot the next transfer overwrites.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | (((N >> 4) & 3) << 14));
}

template <int MT, bool SILU>
__global__ __launch_bounds__(256) void skinny_gemm_kernel(Args a) {
  using Cf = Cfg<MT>;
  constexpr int kS = Cf::kStages, kP = kS - 1, LPI = Cf::kLPI;
  __shared__ __align__(16) uint8_t lds[Cf::kLds];
  // after the reduction, past its area: whether this work-group arrived last
  int &last_flag = *reinterpret_cast<int *>(lds + Cf::kLds - 4);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Work-groups go to the 8 XCDs round-robin by linear index: the S splits
  // of a tile take indices 8 apart and share an XCD.
  const int L = blockIdx.x, r = L / 8;
  const int s = r % a.S;
  const int tile = L % 8 + 8 * (r / a.S);
  if (tile >= a.tiles) return;
  const int n0 = tile * kNT;
  const int steps = a.steps;
  const int kbeg = s * steps * kKS;

  // this lane's transfer sources (the step's k offset is added per issue)
  const uint16_t *wsrc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * (4 * wave + j) + (lane >> 3);  // 1 KiB = 8 rows of W
    const int c = (lane & 7) ^ w_swz(row);
    wsrc[j] = a.W + (long long)(kbeg + row) * a.N + n0 + 8 * c;
  }
  const uint16_t *asrc[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const int row = 4 * (wave * MT + j) + (lane >> 4);  // 1 KiB = 4 rows of A
    const int c = (lane & 15) ^ (row & 15);
    asrc[j] = a.A + (long long)min(row, a.M - 1) * a.K + kbeg + 8 * c;
  }
  auto issue = [&](int u) {
    uint8_t *st = lds + (u % kS) * Cf::kStage;
    const long long wo = (long long)u * kKS * a.N;
    const int ao = u * kKS;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(wsrc[j] + wo, (CFA_LDS void *)(st + 1024 * (4 * wave + j)));
#pragma unroll
    for (int j = 0; j < MT; ++j)
      dma16(asrc[j] + ao, (CFA_LDS void *)(st + kWBytes + 1024 * (wave * MT + j)));
  };

  // operand read offsets within a stage
  const int g = lane >> 4, col = lane & 15;
  const int vrow = 8 * g + (col >> 2);  // rows vrow and vrow + 4 of the wave's k-slice
  const int vh = w_swz(vrow) >> 1;
  const int wbase = (32 * wave + vrow) * (kNT * 2) + ((col >> 1) & 1) * 16 + (col & 1) * 8;
  int boff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) boff[j] = wbase + ((j ^ vh) << 5);
  int aoff[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) aoff[i] = kWBytes + (16 * i + col) * (kKS * 2) + (((4 * wave + g) ^ col) << 4);

  f32x4 acc[MT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int u = 0; u < min(kP, steps); ++u) issue(u);
  for (int t = 0; t < steps; ++t) {
    const int later = min(kP - 1, steps - 1 - t);  // stages issued after this one
    if (later >= 2) wait_vm_lgkm0<2 * LPI>();
    else if (later == 1) wait_vm_lgkm0<LPI>();
    else wait_vm_lgkm0<0>();
    block_barrier();  // every wave's part of stage t has landed
    // the slot refilled here was last read in step t - 1
    if (t + kP < steps) issue(t + kP);
    const uint8_t *st = lds + (t % kS) * Cf::kStage;
    bf16x8 bfr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((CFA_LDS i16x4 *)(st + boff[j]));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((CFA_LDS i16x4 *)(st + boff[j] + 4 * kNT * 2));
      bfr[j] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const bf16x8 af = *reinterpret_cast<const bf16x8 *>(st + aoff[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[j], acc[i][j], 0, 0, 0);
    }
  }

  // the four waves' sums: block (i, j) of wave w at f32x4 index
  // (w * 4 MT + 4 i + j) * 64 + lane; wave w then owns column block j = w
  wait_vm_lgkm0<0>();
  block_barrier();  // every wave is done reading the ring
  f32x4 *red = reinterpret_cast<f32x4 *>(lds);
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[(wave * 4 * MT + 4 * i + j) * 64 + lane] = acc[i][j];
  __syncthreads();
  f32x4 sum[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    sum[i] = red[(4 * i + wave) * 64 + lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) sum[i] += red[(w * 4 * MT + 4 * i + wave) * 64 + lane];
  }

  // sum[i][e] is C[16 i + 4 g + e][n0 + 16 wave + col]
  const int ccol = n0 + 16 * wave + col;
  auto store_c = [&](const f32x4 (&v)[MT]) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * i + 4 * g + e;
        if (row < a.M) a.C[(long long)row * a.N + ccol] = __builtin_bit_cast(uint16_t, (__bf16)v[i][e]);
      }
  };
  // SILU: tile t of W holds gate features 32t .. 32t + 31 in its columns
  // 0..31 and the matching up features in 32..63, so wave w < 2 pairs its
  // gate block with wave w + 2's up block (exchanged through LDS) and
  // writes out[row][32t + 16w + col].
  auto finish = [&](const f32x4 (&v)[MT]) {
    if (!SILU) {
      store_c(v);
      return;
    }
    __syncthreads();  // the reduction's LDS reads are done
    f32x4 *xch = reinterpret_cast<f32x4 *>(lds);
    if (wave >= 2) {
#pragma unroll
      for (int i = 0; i < MT; ++i) xch[((wave - 2) * MT + i) * 64 + lane] = v[i];
    }
    __syncthreads();
    if (wave < 2) {
      const int F = a.N / 2;
      const int fcol = (n0 / 2) + 16 * wave + col;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const f32x4 up = xch[(wave * MT + i) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * i + 4 * g + e;
          if (row >= a.M) continue;
          a.C[(long long)row * F + fcol] = silu_gate(v[i][e], up[e]);
        }
      }
    }
  };
  if (a.S == 1) {
    finish(sum);
    return;
  }
  // Partials cross XCDs, whose L2s are not coherent with each other: they
  // are written and read with device-scope stores and loads (which go to
  // the device's coherence point, not the local L2), in the layout
  // [tile][split][block 4 i + w][element e][lane] so each instruction
  // touches 256 contiguous bytes.  Every store of this work-group has
  // completed (vmcnt 0) before the barrier that precedes its arrival.
  float *mine = a.part + ((long long)tile * a.S + s) * (4 * MT * 256);
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      __hip_atomic_store(mine + ((4 * i + wave) * 4 + e) * 64 + lane, sum[i][e], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0)
    last_flag = __hip_atomic_fetch_add(a.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.S - 1;
  __syncthreads();
  if (!last_flag) return;
  const float *all = a.part + (long long)tile * a.S * (4 * MT * 256);
  for (int q = 0; q < a.S; ++q) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = __hip_atomic_load(all + (long long)q * (4 * MT * 256) + ((4 * i + wave) * 4 + e) * 64 + lane,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sum[i][e] = q == 0 ? v : sum[i][e] + v;
      }
  }
  finish(sum);
  if (tid == 0) __hip_atomic_store(a.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

inline int m_tiles(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8; }

// Splits of K: the largest divisor S of the step count that keeps at most
// one work-group per CU and at least 4 pipeline steps per split.  Measured
// at the draft's shapes (M = 8..128, K = 2048 / 8192, N = 2048..16384) this
// is the fastest split count in every case: more splits add a partial
// round trip and per-work-group start-up latency without adding bandwidth.
inline int default_splits(int N, int K, int cus) {
  const int tiles = N / kNT, steps = K / kKS;
  int best = 1;
  for (int S = 2; S <= steps / 4; ++S)
    if (steps % S == 0 && (long long)tiles * S <= cus) best = S;
  return best;
}

// Workspace: arrival counters for up to kMaxTiles column tiles at a fixed
// offset (so calls of any shape can share one workspace), then the partials.
constexpr int kMaxTiles = 16384;
constexpr size_t kCounterBytes = (size_t)kMaxTiles * 4;

inline size_t workspace_bytes(int M, int N, int S) {
  if (S <= 1) return 0;
  return kCounterBytes + (size_t)(N / kNT) * S * 4 * m_tiles(M) * 1024;
}

}  // namespace sg
}  // namespace cfa

extern "C" size_t cfa_gemm_bf16_skinny_workspace_size(int M, int N, int K, int splits) {
  if (M <= 0 || M > cfa::sg::kMaxM || N <= 0 || N % cfa::sg::kNT || K <= 0 || K % cfa::sg::kKS)
    return 0;
  const int S = splits > 0 ? splits : cfa::sg::default_splits(N, K, cfa::abi::device_cu_count());
  return cfa::sg::workspace_bytes(M, N, S);
}

static int skinny_launch(const void *a, const void *w, void *c, int M, int N, int K, int splits,
                         void *workspace, size_t workspace_bytes, void *stream, bool silu) {
  using namespace cfa::abi;
  namespace sg = cfa::sg;
  clear_error();
  if (M <= 0 || M > sg::kMaxM) return fail_arg("M must be in 1..128");
  if (N <= 0 || N % sg::kNT) return fail_arg("N must be a positive multiple of 64");
  if (K <= 0 || K % sg::kKS) return fail_arg("K must be a positive multiple of 128");
  if (!a || !w || !c) return fail_arg("null pointer");
  if ((((uintptr_t)a | (uintptr_t)w | (uintptr_t)c) & 15) != 0)
    return fail_arg("a, w and c must be 16-byte aligned");
  const int steps = K / sg::kKS;
  const int S = splits > 0 ? splits : sg::default_splits(N, K, device_cu_count());
  if (S > steps || steps % S) return fail_arg("splits must divide K / 128");
  sg::Args g{};
  g.A = (const uint16_t *)a;
  g.W = (const uint16_t *)w;
  g.C = (uint16_t *)c;
  g.M = M;
  g.N = N;
  g.K = K;
  g.S = S;
  g.tiles = N / sg::kNT;
  g.steps = steps / S;
  if (S > 1) {
    if (!workspace || workspace_bytes < sg::workspace_bytes(M, N, S))
      return fail_arg("workspace smaller than cfa_gemm_bf16_skinny_workspace_size");
    if ((uintptr_t)workspace & 255) return fail_arg("workspace must be 256-byte aligned");
    if (g.tiles > sg::kMaxTiles) return fail_arg("N / 64 exceeds 16384 with splits > 1");
    g.cnt = (int *)workspace;
    g.part = (float *)((uint8_t *)workspace + sg::kCounterBytes);
  }
  const long long blocks = (long long)(g.tiles + 7) / 8 * 8 * S;
  if (blocks > 0x7fffffffLL) return fail_arg("problem too large");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks), block(256);
#define CFA_SKINNY(MT)                                                                         \
  do {                                                                                         \
    if (silu)                                                                                  \
      CFA_LAUNCH("gemm_bf16_skinny", (sg::skinny_gemm_kernel<MT, true>), grid, block, 0, st, g);  \
    else                                                                                       \
      CFA_LAUNCH("gemm_bf16_skinny", (sg::skinny_gemm_kernel<MT, false>), grid, block, 0, st, g); \
  } while (0)
  switch (sg::m_tiles(M)) {
    case 1: CFA_SKINNY(1); break;
    case 2: CFA_SKINNY(2); break;
    case 4: CFA_SKINNY(4); break;
    default: CFA_SKINNY(8); break;
  }
#undef CFA_SKINNY
  return CFA_OK;
}

extern "C" int cfa_gemm_bf16_skinny(const void *a, const void *w, void *c, int M, int N, int K,
                                    int splits, void *workspace, size_t workspace_bytes,
                                    void *stream) {
  return skinny_launch(a, w, c, M, N, K, splits, workspace, workspace_bytes, stream, false);
}

extern "C" int cfa_gemm_bf16_skinny_silu(const void *a, const void *w, void *out, int M, int N,
                                         int K, int splits, void *workspace,
                                         size_t workspace_bytes, void *stream) {
  return skinny_launch(a, w, out, M, N, K, splits, workspace, workspace_bytes, stream, true);
}
