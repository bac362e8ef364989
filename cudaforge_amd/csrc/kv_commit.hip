// kv_commit.hip -- commit the accepted draft-tree path into the paged KV cache.
//
// After verification, sequence b keeps the nodes path[0..L) of its draft tree
// (path[0] = 0, the root; node ids increase along a root-to-leaf path).  Their
// K and V, written at slots ctx + path[j] while the tree was verified, move to
// slots ctx + j for every layer and KV head, so that the cache holds the
// accepted tokens contiguously and the next step appends after ctx + L.
// The reference has the metadata half of this (append_tokens,
// csrc/src/memory/paged_kv_cache.cpp:255-286; the context length rule :359-364)
// but no device-side move; the pool layout is paged_kv_cache.cpp:13-21, 409-421:
//   pool[block][layer][kv_head][slot][head_dim].
//
// Hazard: a destination slot j can be the source of an earlier path entry
// (path[j'] = j for j' < j), but never of a later one (path[j'] >= j' > j).
// So a thread that moves one 16-byte column (KV head, chunk, K or V) of the
// rows in increasing j order reads every source before anything overwrites
// it; a batch of rows is read before the batch is written.  One work-group
// per (sequence, layer) checks the path once, one thread per entry.  Rows
// with path[j] == j (the root, and any prefix of a chain) are already in
// place and are neither read nor written; the others are compacted in path
// order, so the batches hold only rows that move.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "abi_internal.hpp"

namespace cfa {
namespace commit {

constexpr int kNT = 256;
constexpr int kMaxPath = 64;
constexpr int kMaxRowBytes = 512;  // head_dim * element size

struct Args {
  uint8_t *kpool, *vpool;
  const int32_t *bt;
  const int32_t *ctx;
  const int32_t *paths;
  const int32_t *plen;
  int32_t *new_ctx;
  int32_t *status;  // per sequence: 0 ok, 1 rejected (bad path or page)
  int max_blocks, num_blocks, num_layers, Hkv, bs, row_bytes, path_stride, B;
};

// Byte offset of (sequence b, slot pos) in layer 0, head 0, or -1 when the
// page is outside the table or the pool.
__device__ __forceinline__ long long slot_base(const Args &a, int b, int pos) {
  const int page = pos / a.bs;
  if (pos < 0 || page >= a.max_blocks) return -1;
  const int blk = a.bt[(long long)b * a.max_blocks + page];
  if (blk < 0 || blk >= a.num_blocks) return -1;
  return ((long long)blk * a.num_layers * a.Hkv * a.bs + pos % a.bs) * (long long)a.row_bytes;
}

constexpr int kBatch = 8;  // rows held in registers per thread at a time
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kNT) void commit_kernel(Args a) {
  __shared__ long long src[kMaxPath], dst[kMaxPath];  // the rows that move, in path order
  __shared__ int n_moves;
  const int layer = blockIdx.x, b = blockIdx.y;
  const int ctx = a.ctx[b];
  const int L = a.plen[b];
  const int32_t *p = a.paths + (long long)b * a.path_stride;
  // path check, one thread per entry of wave 0 (L <= 64): 1 <= L <= kMaxPath,
  // path[0] == 0, strictly increasing, every source and destination slot
  // mapped; the entries with path[j] != j are then compacted in order
  bool good = true;
  const bool shape_ok = L >= 1 && L <= kMaxPath && L <= a.path_stride && ctx >= 0;
  if (threadIdx.x < 64) {
    const int j = threadIdx.x;
    bool moves = false;
    long long so = -1, d = -1;
    if (shape_ok && j < L) {
      const int pj = p[j];
      good = (j == 0) ? (pj == 0) : (pj > p[j - 1]);
      so = slot_base(a, b, ctx + pj);
      d = slot_base(a, b, ctx + j);
      good = good && so >= 0 && d >= 0;
      moves = pj != j;
    }
    const unsigned long long m = __ballot(moves);
    if (moves) {
      const int at = __popcll(m & ((1ull << j) - 1ull));
      src[at] = so;
      dst[at] = d;
    }
    if (j == 0) n_moves = __popcll(m);
  }
  const bool ok = __syncthreads_and(good ? 1 : 0) && shape_ok;
  if (layer == 0 && threadIdx.x == 0) {
    if (a.status) a.status[b] = ok ? 0 : 1;
    if (a.new_ctx) a.new_ctx[b] = ok ? ctx + L : ctx;
  }
  if (!ok) return;
  const int M = n_moves;
  const int cpr = a.row_bytes / 16;  // 16-byte chunks per row
  const long long head_stride = (long long)a.bs * a.row_bytes;
  const long long layer_off = (long long)layer * a.Hkv * head_stride;
  for (int col = threadIdx.x; col < a.Hkv * cpr * 2; col += kNT) {
    const int kv = col / (a.Hkv * cpr), h = (col / cpr) % a.Hkv, c = col % cpr;
    uint8_t *pool = kv ? a.vpool : a.kpool;
    const long long off = layer_off + h * head_stride + 16LL * c;
    for (int j0 = 0; j0 < M; j0 += kBatch) {
      // every load of a batch before any store of it; past the last move a
      // batch repeats that move (the same bytes to the same place), so that
      // loads and stores are unconditional and the batch stays in registers
      // (a clang vector type: an array of HIP's uint4 struct is kept in
      // scratch memory by the compiler)
      u32x4 v[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q)
        v[q] = *reinterpret_cast<const u32x4 *>(pool + src[min(j0 + q, M - 1)] + off);
#pragma unroll
      for (int q = 0; q < kBatch; ++q)
        *reinterpret_cast<u32x4 *>(pool + dst[min(j0 + q, M - 1)] + off) = v[q];
    }
  }
}

}  // namespace commit
}  // namespace cfa

using namespace cfa;

extern "C" int cfa_kv_commit(void *k_pool, void *v_pool, const int32_t *block_tables,
                             int max_blocks_per_seq, const int32_t *ctx_lens,
                             const int32_t *paths, int path_stride, const int32_t *path_lens,
                             int B, int num_blocks, int num_layers, int n_kv_heads,
                             int block_size, int head_dim, int elem_bytes,
                             int32_t *new_ctx_lens, int32_t *status, void *stream) {
  using namespace cfa::abi;
  clear_error();
  if (!k_pool || !v_pool || !block_tables || !ctx_lens || !paths || !path_lens)
    return fail_arg("null pointer argument");
  if (B <= 0 || num_blocks <= 0 || num_layers <= 0 || n_kv_heads <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0)
    return fail_arg("B, num_blocks, num_layers, n_kv_heads, block_size, max_blocks must be positive");
  const long long row = (long long)head_dim * elem_bytes;
  if (head_dim <= 0 || elem_bytes <= 0 || row % 16 || row > commit::kMaxRowBytes)
    return fail_arg("head_dim * elem_bytes must be a multiple of 16 and at most 512");
  if (path_stride < 1) return fail_arg("path_stride must be positive");
  if ((((uintptr_t)k_pool | (uintptr_t)v_pool) & 15) != 0) return fail_arg("pools must be 16-byte aligned");
  if (B > 65535) return fail_arg("B must be at most 65535");
  commit::Args a{};
  a.kpool = (uint8_t *)k_pool;
  a.vpool = (uint8_t *)v_pool;
  a.bt = block_tables;
  a.ctx = ctx_lens;
  a.paths = paths;
  a.plen = path_lens;
  a.new_ctx = new_ctx_lens;
  a.status = status;
  a.max_blocks = max_blocks_per_seq;
  a.num_blocks = num_blocks;
  a.num_layers = num_layers;
  a.Hkv = n_kv_heads;
  a.bs = block_size;
  a.row_bytes = (int)row;
  a.path_stride = path_stride;
  a.B = B;
  CFA_LAUNCH("kv_commit", commit::commit_kernel, dim3(num_layers, B), dim3(commit::kNT), 0,
             (hipStream_t)stream, a);
  return CFA_OK;
}
