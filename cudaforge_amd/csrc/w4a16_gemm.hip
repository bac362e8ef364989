// w4a16_gemm.hip -- fused W4A16 GEMM for many rows (bf16 activations), the
// target model's projections at the verify step (M = B * tree nodes = 504).
//
// C [M, N] = A [M, K] . W [K, N], W dequantised from the reference's packed
// INT4 format (csrc/include/cudaforge/kernels/dequantize.cuh:12-25,
// tests/unit/test_int4_dequant.py:6-15): word (k / 8, n) of B_quant [K/8, N]
// holds nibble k % 8 at bits 4 (k % 8); fp16 group scales s and optional fp16
// zero points z [K / group, N];  w = bf16((nibble - z) * s) formed in fp32,
// (one fp32 fma, then bf16), within one bf16 step of what
// cfa_w4a16_dequant writes, so the result equals dequantise-then-GEMM up to
// that and the order of the fp32 accumulation.
//
// Work-group: a 256 x 256 output tile, eight waves of 128 rows x 64 columns
// (2 x 4), two per SIMD so that one's waits overlap the other's products.
// (A 512 x 128 tile dequantises each weight once, but every work-group then
// re-reads all of A: 0.9 GB per gate/up call, which bounded the kernel.)  K runs in slices of 32 (one
// v_mfma_f32_16x16x32_bf16 k-step).  Everything a slice needs from memory --
// its A tile (256 x 32 bf16), packed words (4 x 256) and scale and zero rows
// -- moves by direct HBM -> LDS transfers into a 3-stage ring, two slices
// ahead; the packed words of slice s + 1 are dequantised once per work-group
// (two words per thread) into one of two [n][k] bf16 tiles while slice s is
// multiplied from the other.  One barrier per slice.  LDS rows of A and of
// the dequantised tiles are 64 bytes; their 16-byte chunks are swizzled by
// row so that the operand reads of 16 lanes (16 rows, one chunk) hit
// distinct banks.
// Split-K (gridDim.z > 1) writes fp32 partials that a second kernel sums in
// split order, so every result is reproducible.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include "abi_internal.hpp"
#include "lds_dma.hpp"
#include "silu.hpp"

namespace cfa {
namespace w4mm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kNT = 64 * kWaves;
constexpr int kBM = 256;             // rows per work-group
constexpr int kBN = 256;             // columns per work-group
constexpr int kWM = 128, kWN = 64;   // rows / columns per wave (2 x 4 waves)
constexpr int kSK = 32;              // k per slice (one MFMA k-step)
constexpr int kMT = kWM / 16;        // 16-row MFMA tiles per wave
constexpr int kNTl = kWN / 16;       // 16-column MFMA tiles per wave
// A moves in stages of two slices (128-byte row segments, one cache line:
// half the requests of one-slice stages), a ring of three
constexpr int kAStages = 3;
constexpr int kARow = 2 * kSK * 2;            // 128 bytes of a row per stage
constexpr int kAStage = kBM * kARow;          // 32 KiB
constexpr int kAXS = kAStage / 1024 / kWaves; // A transfers per wave per stage (4)
constexpr int kAX = kAXS / 2;                 // ... per iteration (2)
constexpr int kWSlots = 6;                    // packed-word ring
constexpr int kQBytes = (kSK / 8) * kBN * 4;  // 4 KiB of packed words per slice
constexpr int kSBytes = kBN * 2;              // one scale row (and one zero row)
constexpr int kWSlot = kQBytes + 2 * kSBytes;
constexpr int kBTile = kBN * kSK * 2;         // one dequantised slice [n][k], 16 KiB
constexpr int kDW = kBN * (kSK / 8) / kNT;    // packed words a thread dequantises per slice (2)
static_assert(kBN == 4 * kWN && kBM == 2 * kWM, "2 x 4 waves");
static_assert(kBN * 2 * 2 == 1024, "one transfer moves the scale and zero rows");
static_assert(kAX == 2, "wait counts below");
#ifndef CFA_W4_SGB
#define CFA_W4_SGB 2
#endif

struct Args {
  const uint16_t *A;   // [M, K] bf16
  const uint32_t *q;   // [K / 8, N]
  const __half *s;     // [K / group, N]
  const __half *z;     // [K / group, N] or null
  uint16_t *C;         // [M, N] bf16
  float *part;         // [splits, M, N] fp32 partials (splits > 1)
  int M, N, K, group;
  int slices_per_split;
  int mtiles;  // row tiles
  int silu;    // C [M, N / 2] = silu(gate) * up, W's columns in the interleaved gate/up layout
  int to_part; // fp32 partials even with one split (the caller sums them)
};

// Byte offset of the 16-byte chunk holding k = 8 c .. 8 c + 7 of a 64-byte
// LDS row r (dequantised tiles): 16 lanes at rows r0 .. r0 + 15 (r0 % 16 ==
// 0) and one chunk hit 16 distinct groups of 4 banks, and so do 8 lanes at
// rows r0 .. r0 + 7 within 128 bytes.  (The earlier swizzle c ^ ((r >> 2) &
// 3) met only the first condition: the dequantised tile's writes, 64 lanes
// at 64 consecutive rows, then took half of the kernel's LDS bank-conflict
// cycles, SQ_LDS_BANK_CONFLICT 7.43M -> 3.70M per gate/up call.)
__host__ __device__ constexpr int sw_off(int r, int c) {
  return r * (kSK * 2) + ((c ^ ((r >> 1) & 3) ^ ((r >> 3) & 1)) << 4);
}
// The same for a 128-byte A row of a stage (chunks 0 .. 7).
__host__ __device__ constexpr int sw_off_a(int r, int c) { return r * kARow + ((c ^ ((r >> 1) & 7)) << 4); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// The 8 weights of one packed word as bf16 pairs (k, k + 1):
// bf16(fma(nibble, s, c)) with c = -z * s, i.e. (nibble - z) * s with one
// fp32 rounding before the bf16 one (cfa_w4a16_dequant rounds the difference
// and the product separately; the two agree to within one bf16 step, far
// inside the GEMM's accumulation-order differences).  Even nibbles are the
// low halves of the bytes of w & 0x0f0f0f0f and odd ones of
// (w >> 4) & 0x0f0f0f0f, so each converts with one byte-to-float
// instruction; each pair packs with one conversion.
//
// Byte P of v as a float: v_cvt_f32_ubyte<P>, written out because the
// compiler otherwise extracts each masked nibble with a bitfield extract
// before converting byte 0 (12 more vector instructions per slice).
template <int P>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
  float r;
  asm("v_cvt_f32_ubyte%2 %0, %1" : "=v"(r) : "v"(v), "i"(P));
  return r;
}
template <int P>
__device__ __forceinline__ uint32_t dequant_pair(uint32_t lo, uint32_t hi, float s, float c) {
  const float f0 = __builtin_fmaf(ubyte_f32<P>(lo), s, c);
  const float f1 = __builtin_fmaf(ubyte_f32<P>(hi), s, c);
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{f0, f1}, bf16x2));
}
__device__ __forceinline__ uint4 dequant_word(uint32_t w, float s, float c) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  return make_uint4(dequant_pair<0>(lo, hi, s, c), dequant_pair<1>(lo, hi, s, c),
                    dequant_pair<2>(lo, hi, s, c), dequant_pair<3>(lo, hi, s, c));
}

// vmcnt(N) lgkmcnt(0)
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | (((N >> 4) & 3) << 14));
}

__global__ __launch_bounds__(kNT, 1) void w4mm_kernel(Args a) {
  __shared__ __align__(16) uint8_t aring[kAStages * kAStage];
  __shared__ __align__(16) uint8_t wring[kWSlots * kWSlot];
  __shared__ __align__(16) uint8_t btile[2][kBTile];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  // the row tiles of one column tile take linear indices 8 apart: one XCD
  // (work-groups go to the 8 XCDs round-robin), whose L2 then serves their
  // common packed weights
  const int L = blockIdx.x, mt = a.mtiles;
  const int ntile = (L % 8) + 8 * (L / (8 * mt)), mti = (L / 8) % mt;
  if (ntile >= a.N / kBN) return;  // padding of the last group of 8 column tiles
  const int n0 = ntile * kBN, mb = mti * kBM;
  const int nsl = a.K / kSK;
  const int s0 = blockIdx.z * a.slices_per_split;
  const int s1 = min(nsl, s0 + a.slices_per_split);
  const int g = lane >> 4, col = lane & 15;
  if (s0 >= s1) return;  // (never: the host sizes the splits) -- uniform per work-group

  // Slices are counted from s0 (relative slice r = absolute s0 + r), so the
  // two slices of A stage t are r = 2t, 2t + 1 whatever s0 is.  Indices past
  // the split are clamped to its last slice: a repeat transfer rewrites the
  // same bytes in place, keeping every wave's transfer count per iteration
  // fixed (the waits below count transfers).
  const int nr = s1 - s0;
  auto abs_slice = [&](int r) { return s0 + min(r, nr - 1); };

  // A transfer x of a stage covers its rows 8 x .. 8 x + 7: lane i lands at
  // row 8 x + i / 8, chunk position i % 8, and so fetches chunk
  // (i % 8) ^ ((row / 2) % 8) of that row -- slice 2t + chunk / 4, k offset
  // 8 (chunk % 4) (rows past M re-read row M - 1).  This wave's transfers
  // of a stage are x = 4 wave .. 4 wave + 3, two per iteration.
  // (element offsets into A, 32-bit: M * K < 2^31 is checked on the host;
  // bit j of ahi: transfer j's chunk lies in the stage's second slice)
  uint32_t aoffs[kAXS];
  uint32_t ahi = 0;
#pragma unroll
  for (int j = 0; j < kAXS; ++j) {
    const int row = 8 * (wave * kAXS + j) + (lane >> 3);
    const int ch = (lane & 7) ^ ((row >> 1) & 7);
    aoffs[j] = (uint32_t)min(mb + row, a.M - 1) * (uint32_t)a.K + 8u * (uint32_t)(ch & 3);
    ahi |= (uint32_t)(ch >> 2) << j;
  }
  // half h (0 or 1) of A stage t
  auto issue_a = [&](int t, int h) {
    uint8_t *dst = aring + (t % kAStages) * kAStage;
    const uint32_t k0 = (uint32_t)abs_slice(2 * t) * kSK, k1 = (uint32_t)abs_slice(2 * t + 1) * kSK;
#pragma unroll
    for (int jj = 0; jj < kAX; ++jj) {
      const int j = 2 * h + jj;
      const uint32_t off = aoffs[j] + (((ahi >> j) & 1u) ? k1 : k0);
      dma16_s(a.A, 2u * off, (CFA_LDS void *)(dst + 1024 * (wave * kAXS + j)));  // M * K < 2^31
    }
  };
  // the word-ring transfer of each wave: waves 0-3 packed row w of the slice
  // (lane: words 4 lane ..), wave 4 the scale row (lanes < 32) and the zero
  // row (lanes >= 32), 8 columns per lane; waves 5-7 repeat wave 0's (the
  // same bytes to the same place), so that every wave issues one word-ring
  // transfer and then kAX A transfers per iteration
  const int ww = wave >= 5 ? 0 : wave;
  const uint32_t qoff = 4u * (uint32_t)((ww & 3) * a.N + n0 + 4 * lane);  // bytes from the slice's row 0
  const __half *ssrc = (lane >= 32 && a.z ? a.z : a.s) + n0 + 8 * (lane & 31);
  auto issue_w = [&](int r) {
    uint8_t *dst = wring + (((r % kWSlots) + kWSlots) % kWSlots) * kWSlot;
    const int k0 = abs_slice(r) * kSK;
    if (ww < 4)
      dma16_s(a.q + (long long)(k0 / 8) * a.N, qoff, (CFA_LDS void *)(dst + 1024 * ww));
    else
      dma16(ssrc + (long long)(k0 / a.group) * a.N, (CFA_LDS void *)(dst + kQBytes));
  };

  // this thread's dequantisation share: column dc, packed rows kDW dp ..
  // kDW dp + kDW - 1 of a slice
  const int dc = tid & (kBN - 1), dp = tid / kBN;
  // without zero points the zero row holds the scales again, multiplied by 0
  // here (scales are finite), so that no branch splits the loop body
  const float zmul = a.z != nullptr ? 1.0f : 0.0f;
  auto words_of = [&](int r, uint32_t (&w)[kDW], float &sf, float &zf) {
    const uint8_t *st = wring + (min(r, nr - 1) % kWSlots) * kWSlot;
#pragma unroll
    for (int j = 0; j < kDW; ++j)
      w[j] = *reinterpret_cast<const uint32_t *>(st + ((kDW * dp + j) * kBN + dc) * 4);
    const __half *sc = reinterpret_cast<const __half *>(st + kQBytes);
    sf = __half2float(sc[dc]);
    zf = -(__half2float(sc[kBN + dc]) * zmul) * sf;  // the fma's addend -z * s
  };

  f32x4 acc[kMT][kNTl];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kNTl; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // operand read offsets of this lane (A: slice half 0 of a stage; half 1 is
  // chunk + 4, i.e. the byte offset with bit 6 flipped)
  // (rows 16 i apart share the swizzle, so tile i is tile 0 + 2048 i bytes;
  // B tile j is tile 0 + 1024 j bytes)
  const int aoff0 = sw_off_a(wm * kWM + col, g), boff0 = sw_off(wn * kWN + col, g);
  static_assert(sw_off_a(16, 0) == 16 * kARow && sw_off(16, 0) == 16 * kSK * 2, "offsets");

  // Pipeline, per iteration r: after the barrier, A of slice r + 1 and the
  // dequantised tile of slice r + 1 are complete; this wave issues W(r + 5)
  // and half r % 2 of A stage r / 2 + 2, reads slice r + 1's operands into
  // its spare registers, dequantises slice r + 2 into the tile slice r used,
  // and multiplies slice r from the registers read one iteration earlier --
  // so the MFMAs never wait for LDS.  The prologue issues W(0), then for the
  // virtual iterations r = -4 .. -1 the same pairs: W(1 .. 4), A stages 0
  // and 1.  At the top of iteration r every transfer of iterations <= r - 2
  // has landed once at most the 1 + kAX transfers of iteration r - 1 are in
  // flight: among them the whole stage of slice r + 1 (its second half was
  // issued at iteration 2 ((r + 1) / 2) - 3 <= r - 2) and W(r + 2) (issued
  // at r - 3).  A stage t goes to slot t % 3 at iteration 2 t - 4, after the
  // operands of stage t - 3 were read (iterations <= 2 t - 6).
  issue_w(0);
#pragma unroll
  for (int r = -4; r < 0; ++r) {
    issue_w(r + 5);
    issue_a((r >> 1) + 2, r & 1);
  }
  auto dequant_into = [&](int r) {
    uint32_t w[kDW];
    float sf, zf;
    words_of(r, w, sf, zf);
#pragma unroll
    for (int j = 0; j < kDW; ++j)
      *reinterpret_cast<uint4 *>(btile[r & 1] + sw_off(dc, kDW * dp + j)) = dequant_word(w[j], sf, zf);
  };
  bf16x8 a0[kMT], b0[kNTl], a1[kMT], b1[kNTl];
  auto read_ops = [&](int r, bf16x8 (&af)[kMT], bf16x8 (&bf)[kNTl]) {
    r = min(r, nr - 1);
    const uint8_t *as = aring + ((r >> 1) % kAStages) * kAStage + (aoff0 ^ ((r & 1) << 6));
    const uint8_t *bs = btile[r & 1] + boff0;
#pragma unroll
    for (int j = 0; j < kNTl; ++j) bf[j] = *reinterpret_cast<const bf16x8 *>(bs + 1024 * j);
#pragma unroll
    for (int i = 0; i < kMT; ++i) af[i] = *reinterpret_cast<const bf16x8 *>(as + 2048 * i);
  };
  wait_vm_lgkm0<kAX + 3 * (1 + kAX)>();  // W(0), W(1)
  block_barrier();
  dequant_into(0);
  dequant_into(1);
  wait_vm_lgkm0<2 * (1 + kAX)>();  // A stage 0; and the dequantised writes
  block_barrier();
  read_ops(0, a0, b0);

  auto step = [&](int r, bf16x8 (&ac)[kMT], bf16x8 (&bc)[kNTl], bf16x8 (&an)[kMT],
                  bf16x8 (&bn)[kNTl]) {
    wait_vm_lgkm0<1 + kAX>();
    block_barrier();
    issue_w(r + 5);
    issue_a((r >> 1) + 2, r & 1);
    read_ops(r + 1, an, bn);
    dequant_into(r + 2);
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int j = 0; j < kNTl; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac[i], bc[j], acc[i][j], 0, 0, 0);
#if CFA_W4_SGB
    // LDS reads first (the next slice's operands, the words), then the
    // dequantisation's VALU work spread between the MFMAs, so that the two
    // waves of a SIMD (which reach this point together) overlap VALU with
    // products instead of taking turns; its LDS writes last
    __builtin_amdgcn_sched_group_barrier(0x0100, kNTl + kMT + 2 * kDW + 2, 0);
#pragma unroll
    for (int k = 0; k < kMT * kNTl; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x0002, CFA_W4_SGB, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x0200, kDW, 0);
#endif
  };
  int r = 0;
  for (; r + 1 < nr; r += 2) {
    step(r, a0, b0, a1, b1);
    step(r + 1, a1, b1, a0, b0);
  }
  if (r < nr) step(r, a0, b0, a1, b1);
  // drain: the last iterations' repeat transfers must land before exit
  wait_vm_lgkm0<0>();

  // acc[i][j][e]: row mb + 128 wm + 16 i + 4 g + e, column n0 + 64 wn + 16 j + lane % 16
  const int r0 = mb + wm * kWM + 4 * g, c0 = n0 + wn * kWN + col;
  const bool to_part = gridDim.z > 1 || a.to_part;
  if (!to_part && a.silu) {
    // this wave's 64 columns are gate features f .. f + 31 (tiles j = 0, 1)
    // and then their up columns (j = 2, 3): a lane holds both halves of its
    // features
    const int F = a.N / 2, f0 = (n0 + wn * kWN) / 2 + col;
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + 16 * i + e;
        if (row >= a.M) continue;
        uint16_t *cr = a.C + (long long)row * F + f0;
        static_assert(kNTl == 4, "two gate and two up tiles per wave");
        const uint32_t p = silu_gate2(acc[i][0][e], acc[i][2][e], acc[i][1][e], acc[i][3][e]);
        cr[0] = (uint16_t)p;
        cr[16] = (uint16_t)(p >> 16);
      }
  } else if (!to_part) {
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + 16 * i + e;
        if (row >= a.M) continue;
        uint16_t *cr = a.C + (long long)row * a.N + c0;
#pragma unroll
        for (int j = 0; j < kNTl; ++j) cr[16 * j] = __builtin_bit_cast(uint16_t, (__bf16)acc[i][j][e]);
      }
  } else {
    float *pp = a.part + (long long)blockIdx.z * a.M * a.N;
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + 16 * i + e;
        if (row >= a.M) continue;
        float *pr = pp + (long long)row * a.N + c0;
#pragma unroll
        for (int j = 0; j < kNTl; ++j) pr[16 * j] = acc[i][j][e];
      }
  }
}

// C = bf16(sum of the split partials in split order), four columns per thread.
__global__ __launch_bounds__(256) void w4mm_reduce_kernel(const float *part, uint16_t *C, long long MN,
                                                          int splits) {
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= MN) return;
  float4 acc = *reinterpret_cast<const float4 *>(part + i);
  for (int s = 1; s < splits; ++s) {
    const float4 v = *reinterpret_cast<const float4 *>(part + (long long)s * MN + i);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  uint2 o;
  o.x = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc.x) |
        ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc.y) << 16);
  o.y = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc.z) |
        ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc.w) << 16);
  *reinterpret_cast<uint2 *>(C + i) = o;
}

// The same for the SiLU-gated output: four features f .. f + 3 per thread
// (gate columns 64 (f / 32) + f % 32 .., up columns 32 further on).
__global__ __launch_bounds__(256) void w4mm_reduce_silu_kernel(const float *part, uint16_t *C, int M,
                                                               int N, int splits) {
  const int F = N / 2;
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= (long long)M * F) return;
  const long long m = i / F;
  const int f = (int)(i % F);
  const long long gi = m * N + 64 * (f / 32) + f % 32, MN = (long long)M * N;
  float4 gs = *reinterpret_cast<const float4 *>(part + gi);
  float4 us = *reinterpret_cast<const float4 *>(part + gi + 32);
  for (int s = 1; s < splits; ++s) {
    const float4 g = *reinterpret_cast<const float4 *>(part + s * MN + gi);
    const float4 u = *reinterpret_cast<const float4 *>(part + s * MN + gi + 32);
    gs.x += g.x;
    gs.y += g.y;
    gs.z += g.z;
    gs.w += g.w;
    us.x += u.x;
    us.y += u.y;
    us.z += u.z;
    us.w += u.w;
  }
  uint2 o;
  o.x = silu_gate2(gs.x, us.x, gs.y, us.y);
  o.y = silu_gate2(gs.z, us.z, gs.w, us.w);
  *reinterpret_cast<uint2 *>(C + i) = o;
}

// Splits of K: enough work-groups for every CU, each split at least 8
// slices; *spp slices per split, and no split empty.
int choose_splits(int M, int N, int K, int cus, int *spp) {
  const long long tiles = (long long)((M + kBM - 1) / kBM) * (N / kBN);
  const int nsl = K / kSK;
  // as many splits as fit in one round of work-groups (one per CU)
  const int s = (int)std::max<long long>(1, std::min<long long>({(long long)cus / std::max(tiles, 1LL), (long long)nsl / 8, 16LL}));
  const int per = (nsl + s - 1) / s;
  if (spp) *spp = per;
  return (nsl + per - 1) / per;
}

}  // namespace w4mm
}  // namespace cfa

extern "C" size_t cfa_w4a16_gemm_zp_workspace_size(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % cfa::w4mm::kBN != 0 || K % cfa::w4mm::kSK != 0) return 0;
  const int s = cfa::w4mm::choose_splits(M, N, K, cfa::abi::device_cu_count(), nullptr);
  return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

// mode: 0 bf16 C, 1 SiLU-gated bf16 C, 2 fp32 partials only (in workspace)
static int w4mm_launch(const void *a, const uint32_t *b_quant, const void *scales, const void *zeros,
                       int M, int N, int K, int group_size, void *c, void *workspace,
                       size_t workspace_bytes, void *stream, int mode) {
  const bool silu = mode == 1, part_only = mode == 2;
  using namespace cfa::abi;
  using namespace cfa::w4mm;
  clear_error();
  if (M <= 0 || N <= 0 || K <= 0) return fail_arg("M, N and K must be positive");
  if (N % kBN != 0) return fail_arg("N must be a multiple of 256");
  if (K % kSK != 0) return fail_arg("K must be a multiple of 32");
  if (group_size <= 0 || group_size % kSK != 0 || K % group_size != 0)
    return fail_arg("group_size must be a multiple of 32 that divides K");
  if (!a || !b_quant || !scales || (!c && !part_only)) return fail_arg("null pointer");
  if ((((uintptr_t)a | (uintptr_t)c | (uintptr_t)b_quant | (uintptr_t)scales | (uintptr_t)zeros) & 15) != 0)
    return fail_arg("a, b_quant, scales, zeros and c must be 16-byte aligned");
  int spp = 0;
  if ((long long)M * K >= (1LL << 31)) return fail_arg("M * K must be below 2^31");
  const int splits = choose_splits(M, N, K, device_cu_count(), &spp);
  const size_t need = (splits > 1 || part_only) ? (size_t)splits * M * N * sizeof(float) : 0;
  if (need && (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 15) != 0))
    return fail_arg(part_only ? "part too small (cfa_w4a16_gemm_zp_splits x M x N fp32)"
                              : "workspace too small (see cfa_w4a16_gemm_zp_workspace_size)");
  Args g{};
  g.A = (const uint16_t *)a;
  g.q = b_quant;
  g.s = (const __half *)scales;
  g.z = (const __half *)zeros;
  g.C = (uint16_t *)c;
  g.part = (float *)workspace;
  g.M = M;
  g.N = N;
  g.K = K;
  g.group = group_size;
  g.slices_per_split = spp;
  g.silu = silu ? 1 : 0;
  g.to_part = part_only ? 1 : 0;
  const long long mt = (M + kBM - 1) / kBM;
  if (mt > 65535) return fail_arg("M too large");
  hipStream_t st = (hipStream_t)stream;
  const long long blocks = mt * ((N / kBN + 7) / 8) * 8;  // column tiles padded to groups of 8
  if (blocks > 0x7fffffffLL) return fail_arg("problem too large");
  g.mtiles = (int)mt;
  CFA_LAUNCH(silu ? "w4a16_gemm_zp_silu" : "w4a16_gemm_zp", w4mm_kernel,
             dim3((unsigned)blocks, 1, (unsigned)splits), dim3(kNT), 0, st, g);
  if (part_only) return CFA_OK;
  if (splits > 1 && silu) {
    const long long MF = (long long)M * (N / 2);  // N % 256 == 0: four features per thread
    CFA_LAUNCH("w4a16_gemm_zp_reduce", w4mm_reduce_silu_kernel,
               dim3((unsigned)((MF / 4 + 255) / 256)), dim3(256), 0, st, (const float *)workspace,
               (uint16_t *)c, M, N, splits);
  } else if (splits > 1) {
    const long long MN = (long long)M * N;  // N % 128 == 0: four columns per thread
    CFA_LAUNCH("w4a16_gemm_zp_reduce", w4mm_reduce_kernel, dim3((unsigned)((MN / 4 + 255) / 256)),
               dim3(256), 0, st, (const float *)workspace, (uint16_t *)c, MN, splits);
  }
  return CFA_OK;
}

extern "C" int cfa_w4a16_gemm_zp(const void *a, const uint32_t *b_quant, const void *scales,
                                 const void *zeros, int M, int N, int K, int group_size, void *c,
                                 void *workspace, size_t workspace_bytes, void *stream) {
  return w4mm_launch(a, b_quant, scales, zeros, M, N, K, group_size, c, workspace, workspace_bytes,
                     stream, 0);
}

extern "C" int cfa_w4a16_gemm_zp_silu(const void *a, const uint32_t *b_quant, const void *scales,
                                      const void *zeros, int M, int N, int K, int group_size,
                                      void *c, void *workspace, size_t workspace_bytes,
                                      void *stream) {
  return w4mm_launch(a, b_quant, scales, zeros, M, N, K, group_size, c, workspace, workspace_bytes,
                     stream, 1);
}

extern "C" int cfa_w4a16_gemm_zp_splits(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % cfa::w4mm::kBN != 0 || K % cfa::w4mm::kSK != 0) return 0;
  return cfa::w4mm::choose_splits(M, N, K, cfa::abi::device_cu_count(), nullptr);
}

extern "C" int cfa_w4a16_gemm_zp_partials(const void *a, const uint32_t *b_quant, const void *scales,
                                          const void *zeros, int M, int N, int K, int group_size,
                                          float *part, size_t part_bytes, void *stream) {
  return w4mm_launch(a, b_quant, scales, zeros, M, N, K, group_size, nullptr, part, part_bytes,
                     stream, 2);
}
