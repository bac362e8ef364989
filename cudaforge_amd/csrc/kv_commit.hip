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
// (path[j'] = j for j' < j), so moving in parallel would race.  Each
// work-group owns one (sequence, layer, head) and reads every moved row of K
// and V into LDS before writing any.  Rows with path[j] == j (the root, and
// any prefix of a chain) are already in place and are neither read nor
// written.
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

// Byte offset of (sequence b, slot pos, layer, head) or -1 when the page is
// outside the table or the pool.
__device__ __forceinline__ long long slot_off(const Args &a, int b, int pos, int layer, int h) {
  const int page = pos / a.bs;
  if (pos < 0 || page >= a.max_blocks) return -1;
  const int blk = a.bt[(long long)b * a.max_blocks + page];
  if (blk < 0 || blk >= a.num_blocks) return -1;
  return ((((long long)blk * a.num_layers + layer) * a.Hkv + h) * a.bs + pos % a.bs) *
         (long long)a.row_bytes;
}

// Validity of sequence b's path: 1 <= L <= kMaxPath, path[0] == 0, strictly
// increasing, and every source and destination slot mapped.  Evaluated
// identically by every work-group of the sequence, so a rejected sequence is
// left untouched everywhere.
__device__ bool path_ok(const Args &a, int b, int ctx, int L) {
  if (L < 1 || L > kMaxPath || L > a.path_stride || ctx < 0) return false;
  const int32_t *p = a.paths + (long long)b * a.path_stride;
  if (p[0] != 0) return false;
  for (int j = 1; j < L; ++j)
    if (p[j] <= p[j - 1]) return false;
  for (int j = 0; j < L; ++j)
    if (slot_off(a, b, ctx + p[j], 0, 0) < 0 || slot_off(a, b, ctx + j, 0, 0) < 0) return false;
  return true;
}

__global__ __launch_bounds__(kNT) void commit_kernel(Args a) {
  __shared__ uint4 buf[2][kMaxPath * (kMaxRowBytes / 16)];
  __shared__ int ok;
  const int h = blockIdx.x, layer = blockIdx.y, b = blockIdx.z;
  const int ctx = a.ctx[b];
  const int L = a.plen[b];
  if (threadIdx.x == 0) ok = path_ok(a, b, ctx, L) ? 1 : 0;
  __syncthreads();
  if (h == 0 && layer == 0 && threadIdx.x == 0) {
    if (a.status) a.status[b] = ok ? 0 : 1;
    if (a.new_ctx) a.new_ctx[b] = ok ? ctx + L : ctx;
  }
  if (!ok) return;
  const int32_t *p = a.paths + (long long)b * a.path_stride;
  const int cpr = a.row_bytes / 16;  // 16-byte chunks per row
  const int n = L * cpr;
  // read every moved row (K then V) before writing any
  for (int i = threadIdx.x; i < n; i += kNT) {
    const int j = i / cpr, c = i % cpr;
    if (p[j] == j) continue;
    const long long so = slot_off(a, b, ctx + p[j], layer, h) + 16LL * c;
    buf[0][i] = *reinterpret_cast<const uint4 *>(a.kpool + so);
    buf[1][i] = *reinterpret_cast<const uint4 *>(a.vpool + so);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += kNT) {
    const int j = i / cpr, c = i % cpr;
    if (p[j] == j) continue;
    const long long d = slot_off(a, b, ctx + j, layer, h) + 16LL * c;
    *reinterpret_cast<uint4 *>(a.kpool + d) = buf[0][i];
    *reinterpret_cast<uint4 *>(a.vpool + d) = buf[1][i];
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
  if (B > 65535 || num_layers > 65535) return fail_arg("B and num_layers must be at most 65535");
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
  CFA_LAUNCH("kv_commit", commit::commit_kernel, dim3(n_kv_heads, num_layers, B), dim3(commit::kNT),
             0, (hipStream_t)stream, a);
  return CFA_OK;
}
