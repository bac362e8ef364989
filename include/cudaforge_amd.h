/*
 * cudaforge_amd.h -- C ABI of the MI355X (gfx950) speculative-decoding
 * verification library (libcfa.so).
 *
 * Every entry point takes plain pointers and sizes.  Pointers named as device
 * buffers are HIP device addresses (e.g. torch.Tensor.data_ptr()); `stream` is
 * a hipStream_t (NULL = default stream) and all device work is enqueued on it
 * in order, without host synchronisation.  The library allocates no device
 * memory: scratch space is the caller's `workspace` (cfa_chain_verify_noalloc
 * uses a static device array of the library instead).
 *
 * Errors: every function returns CFA_OK (0) or a negative code; the message
 * of the calling thread's last failure is available from cfa_last_error().
 * CFA_ERR_ARG corresponds to the std::invalid_argument the reference throws
 * (surfaced by its pybind layer as ValueError); CFA_ERR_HIP is a HIP runtime
 * failure.  No C++ exception crosses this boundary.
 *
 * Reference interfaces replaced (paths inside Bahaa-Labs/CUDAForge):
 *   cudaforge/speculative.py:27-217            SpeculativeEngine.step (python)
 *   csrc/include/cudaforge/scheduler/speculative.h:14-88, bound at
 *   csrc/bindings/pybind_module.cpp:196-239    SpeculativeEngine (C++)
 *   csrc/include/cudaforge/memory/paged_kv_cache.h:81-94
 *                                              KVCacheBatchDescriptor layout
 *   csrc/include/cudaforge/memory/paged_kv_cache.h:36-179, bound at
 *   csrc/bindings/pybind_module.cpp:20-99      PagedKVCache (host page tables)
 */
#ifndef CUDAFORGE_AMD_H
#define CUDAFORGE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CFA_OK 0
#define CFA_ERR_ARG (-1)
#define CFA_ERR_HIP (-2)
#define CFA_ERR_STATE (-3)        /* std::runtime_error in the reference */
#define CFA_ERR_RANGE (-4)        /* std::out_of_range in the reference */
#define CFA_ERR_OUT_OF_PAGES (-5) /* OutOfPagesException (paged_kv_cache.h:31-34) */

/* input_kind */
#define CFA_INPUT_PROBS 0  /* rows are probabilities (the C++ engine's input) */
#define CFA_INPUT_LOGITS 1 /* rows are logits; softmax(logits / T) is fused */

/* mode */
#define CFA_MODE_CPP 0    /* per-row rules of speculative.cpp:50-103 */
#define CFA_MODE_PYTHON 1 /* batch lock-step rules of speculative.py:152-195 */
#define CFA_MODE_GREEDY 2 /* speculative.cpp:105-150 */

/* Message of this thread's last failed call ("" if none). */
const char *cfa_last_error(void);

/* Library ABI version (major * 100 + minor); equals CFA_ABI_VERSION for a
 * library built from this header.  Major 2 changed two contracts of major 1:
 * cfa_tree_verify takes (workspace, workspace_bytes) before its stream, and
 * python-mode cfa_chain_verify reads uniforms [B, K+2] (row stride K+2), not
 * [B, K+1].  Binding code checks the major before its first call. */
#define CFA_ABI_VERSION 200
int cfa_version(void);

/* ---------------------------------------------------------------------------
 * Chain verification.
 *
 * Replaces SpeculativeEngine::verify_candidates / verify_candidates_greedy
 * (speculative.h:56-68, speculative.cpp:50-150; pybind names at
 * pybind_module.cpp:229-235) for B sequences at once, and the acceptance
 * phase of cudaforge/speculative.py:152-195.
 *
 *   target   [B, K+1, V] fp32, row (b,i) at target + b*t_stride_b + i*t_stride_k
 *   draft    [B, K,   V] fp32, row (b,i) at draft  + b*d_stride_b + i*d_stride_k
 *            (unused in greedy mode)
 *   input_kind  CFA_INPUT_PROBS or CFA_INPUT_LOGITS (softmax of row / temperature)
 *   draft_tokens [B, K] int32 (token ids in [0, V); an id outside that range
 *            is never accepted and never dereferenced)
 *   uniforms fp32 in [0, 1):
 *     CFA_MODE_CPP: [B, K+1], the draws the reference takes from its mt19937,
 *       in order (one per acceptance test, then one for the resample / bonus
 *       draw);
 *     CFA_MODE_PYTHON: [B, K+2]; columns 0..K-1 replace torch.rand_like at
 *       speculative.py:161, column K drives the resample / bonus draw, column
 *       K+1 the bonus that follows a rejection at the last position (there
 *       the reference's num_accepted reaches K, so speculative.py:188 appends
 *       a bonus after the resampled token).  Python-mode draws take the first
 *       index whose sequential fp32 prefix sum exceeds u (never an index of
 *       zero weight, as torch.multinomial), and past the end of the sums the
 *       last index of positive weight.
 *   top_p    nucleus threshold of the python-mode bonus draw (speculative.py:67-81)
 *   eos_token_id  (< 0: none) CFA_MODE_CPP / GREEDY only
 *
 * Outputs (device, int32):
 *   out_accept_len  [B]    accepted draft tokens (the reference's num_accepted;
 *                          python mode: the batch-wide count n, speculative.py:166)
 *   out_tokens      [B, K+1] accepted drafts then the final token, -1 padded
 *                          (python mode, n = K - 1: the K - 1 drafts, the
 *                          resampled token and the bonus)
 *   out_num_emitted [B]    valid entries of out_tokens
 *   out_final       [B]    final_token (resample or bonus draw; the last
 *                          token emitted)
 *   out_eos         [B]    end_of_sequence
 *   out_target_probs / out_draft_probs (optional, may be NULL): contiguous
 *     [B,K+1,V] / [B,K,V] copies of the probabilities the decisions used.
 *
 * The resample / bonus draw reproduces the reference's sequential fp32 inverse
 * CDF (speculative.cpp:11-48) bit for bit.
 */
size_t cfa_chain_verify_workspace_size(int B, int K, int V, int input_kind, int mode);

int cfa_chain_verify(const float *target, int64_t t_stride_b, int64_t t_stride_k,
                     const float *draft, int64_t d_stride_b, int64_t d_stride_k,
                     int input_kind, const int32_t *draft_tokens, const float *uniforms,
                     int B, int K, int V, float temperature, float top_p, int mode,
                     int32_t eos_token_id, int32_t *out_accept_len, int32_t *out_tokens,
                     int32_t *out_num_emitted, int32_t *out_final, int32_t *out_eos,
                     float *out_target_probs, float *out_draft_probs, void *workspace,
                     size_t workspace_bytes, void *stream);

/* cfa_chain_verify without a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops or harnesses that forbid hipMalloc).  Its scratch is
 * a static 32 MiB device array inside the library (one per GPU, held until
 * the process ends); shapes whose cfa_chain_verify_workspace_size exceeds
 * 32 MiB are refused with CFA_ERR_ARG (B = 64, K = 8, V = 128256 needs
 * 18.7 MiB).  It allocates nothing.  Every call on one GPU shares that array,
 * so calls that overlap on one GPU (other streams, other host threads) race;
 * serialise them.  Arguments and results are those of cfa_chain_verify. */
int cfa_chain_verify_noalloc(const float *target, int64_t t_stride_b, int64_t t_stride_k,
                             const float *draft, int64_t d_stride_b, int64_t d_stride_k,
                             int input_kind, const int32_t *draft_tokens, const float *uniforms,
                             int B, int K, int V, float temperature, float top_p, int mode,
                             int32_t eos_token_id, int32_t *out_accept_len, int32_t *out_tokens,
                             int32_t *out_num_emitted, int32_t *out_final, int32_t *out_eos,
                             float *out_target_probs, float *out_draft_probs, void *stream);

/* ---------------------------------------------------------------------------
 * Token sampler: plain decode and draft-tree expansion.
 *
 * Replaces launch_fused_sampling / fused_sampling_kernel
 * (csrc/include/cudaforge/engine/sampling.h:18-28, 61-216) and
 * fused_sampling_triton (csrc/kernels/triton/sampling_triton.py:6-66), and
 * draws the children of draft-tree nodes.  R rows of V values at
 * rows + r * row_stride (logits, or probabilities for CFA_INPUT_PROBS);
 * `draws` tokens per row, out_tokens [R, draws]:
 *   CFA_SAMPLE_MULTINOMIAL  p = softmax(row / temperature); token = first i
 *     with u <= p_0 + ... + p_i summed sequentially in fp32, V - 1 if none
 *     (sampling.h:164-185, speculative.cpp:11-24), one uniform per draw
 *     (uniforms [R, draws]).  top_k / top_p are ignored, as the reference
 *     kernel ignores them.
 *   CFA_SAMPLE_FILTERED  keep p_i >= the top-p threshold of
 *     cudaforge/speculative.py:67-81 and >= the top_k-th largest p (top_k <= 0:
 *     no top-k), renormalise by the kept mass, then the python-mode draw of
 *     cfa_chain_verify (first i whose prefix sum exceeds u, never a token
 *     that was filtered out).
 *   CFA_SAMPLE_GREEDY  the `draws` (<= 8) largest raw values, largest first,
 *     equal values by lower index (sampling.h:107-135 for draws = 1); no
 *     uniforms, no temperature.
 * out_probs [R, V] (optional, not in greedy mode) receives the probabilities
 * the draws used.  Independent draws of one row (draws > 1) sample with
 * replacement: the children of a tree node drawn i.i.d. from its draft
 * distribution, as multi-candidate rejection sampling requires.
 */
#define CFA_SAMPLE_MULTINOMIAL 0
#define CFA_SAMPLE_FILTERED 1
#define CFA_SAMPLE_GREEDY 2

size_t cfa_sample_workspace_size(int R, int V, int draws, int mode);
int cfa_sample(const float *rows, int64_t row_stride, int input_kind, int R, int V, int draws,
               float temperature, int top_k, float top_p, int mode, const float *uniforms,
               int32_t *out_tokens, float *out_probs, void *workspace, size_t workspace_bytes,
               void *stream);

/* ---------------------------------------------------------------------------
 * Tree-masked verification attention over a paged KV cache (bf16, MFMA).
 *
 * No reference kernel exists (the reference's target forward recomputes the
 * whole prefix, cudaforge/speculative.py:139-141); the arguments mirror the
 * reference's paged-cache descriptor KVCacheBatchDescriptor
 * (csrc/include/cudaforge/memory/paged_kv_cache.h:81-94: block_tables,
 * context_lens, max_blocks_per_seq, block_size, num_kv_heads, head_dim, key
 * and value pools) and its pool layout (paged_kv_cache.cpp:13-21, 409-421):
 *   pool[block][layer][kv_head][slot][head_dim]  bf16
 *
 *   head_dim   128 or 64
 *   q          [B, N - first_node, n_q_heads, head_dim] bf16 -- queries of the
 *              tree nodes first_node .. N - 1 (first_node = 0: every node, as
 *              a verify step needs; a drafter growing its tree level by level
 *              passes the newest level)
 *   block_tables [B, max_blocks_per_seq] int32, ctx_lens [B] int32
 *   the tree's own K/V sit at positions ctx_len .. ctx_len + N - 1
 *   tree_mask  uint64 per node (bit j: node j is an ancestor of, or is, the
 *              node), [N] shared (stride 0) or [B, N] (stride N)
 *   max_keys   host-side bound on ctx_len + N over the batch (plans the splits)
 *   num_splits key-range splits (0: automatic); splits > 1 need workspace
 *   out        [B, N - first_node, n_q_heads, head_dim] bf16
 * Query (node i, head hq) attends to context positions [0, ctx_len) and to
 * tree positions ctx_len + j with bit j of tree_mask[i]; scores scale by
 * sm_scale; fp32 softmax and accumulation.  The workspace size takes N as the
 * number of query nodes (N - first_node; the full N is an upper bound).
 */
size_t cfa_tree_attention_workspace_size(int B, int N, int n_q_heads, int n_kv_heads,
                                         int head_dim, int max_keys, int num_splits);

int cfa_tree_attention(const void *q, const void *k_pool, const void *v_pool,
                       const int32_t *block_tables, int max_blocks_per_seq,
                       const int32_t *ctx_lens, int num_blocks, int num_layers, int layer,
                       int block_size, const uint64_t *tree_mask, int64_t tree_mask_stride_b,
                       int B, int N, int first_node, int n_q_heads, int n_kv_heads,
                       int head_dim, float sm_scale, int max_keys, int num_splits, void *out,
                       void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Tree verification: multi-candidate rejection sampling down a draft tree,
 * longest accepted root-to-leaf path and the resample / bonus token.
 *
 * Generalises SpeculativeEngine::verify_candidates / _greedy
 * (csrc/src/scheduler/speculative.cpp:50-150; pybind names at
 * csrc/bindings/pybind_module.cpp:229-235) from a chain of K drafts to a tree
 * of N <= 64 nodes (parents[c] < c, node 0 = root = the last verified token);
 * on a one-child chain it is exactly verify_candidates.
 *
 *   target [B, N, V] fp32: row n = target distribution after node n
 *   draft  [B, N, V] fp32: row n = distribution node n's children were drawn
 *          from (unused in greedy mode); probabilities or logits (input_kind)
 *   parents    [N] shared (stride 0) or [B, N] (stride N) int32
 *   node_tokens [B, N] int32 (the root's entry is not read)
 *   uniforms   [B, n_uniforms]: the stream the walk consumes, one draw per
 *              acceptance test and one for the final draw (as the reference's
 *              mt19937 stream, speculative.cpp:64, 72, 13-14)
 *   mode       CFA_MODE_CPP or CFA_MODE_GREEDY
 * Outputs (int32): path [B, N] accepted node ids from the root, -1 padded;
 * path_len [B] (1 + accepted drafts); tokens [B, N+1] accepted draft tokens
 * then the final token; num_emitted [B]; final [B]; eos [B]; status [B]
 * (optional; 1 when the uniform stream ran out, 2 when a wait between the
 * work-groups of a sequence timed out -- the outputs are then invalid).
 * out_target_probs / out_draft_probs (optional, [B, N, V]) receive the
 * probabilities of the rows the walk visited.
 *
 * Up to 8 work-groups share each sequence (they exchange row statistics and
 * split every exact pass, so they must run together: the launch never holds
 * more work-groups than the device runs at once, and kernels of other streams
 * can only delay a member -- past the bounded wait, status 2; environment
 * CFA_COOPERATIVE_LAUNCH=1 launches with hipLaunchCooperativeKernel, which
 * guarantees residency but slows this call and the process's next
 * dispatches); workspace is
 * cfa_tree_verify_workspace_size(B) bytes, 256-byte aligned, holding their
 * barrier and exchange state (cleared by the call itself).  Calls sharing a
 * workspace must not overlap.
 */
size_t cfa_tree_verify_workspace_size(int B);
int cfa_tree_verify(const float *target, int64_t t_stride_b, int64_t t_stride_n,
                    const float *draft, int64_t d_stride_b, int64_t d_stride_n, int input_kind,
                    const int32_t *parents, int64_t parents_stride_b, const int32_t *node_tokens,
                    const float *uniforms, int n_uniforms, int B, int N, int V,
                    float temperature, int mode, int32_t eos_token_id, int32_t *out_path,
                    int32_t *out_path_len, int32_t *out_tokens, int32_t *out_num_emitted,
                    int32_t *out_final, int32_t *out_eos, int32_t *out_status,
                    float *out_target_probs, float *out_draft_probs, void *workspace,
                    size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * KV commit / compaction of an accepted draft-tree path.
 *
 * Device half of the reference's append_tokens(seq, L)
 * (csrc/src/memory/paged_kv_cache.cpp:255-286; context length :359-364),
 * which the reference performs on host metadata only: for each sequence b the
 * accepted nodes paths[b, 0..L) (paths[b,0] = 0, strictly increasing) move
 * from slots ctx_lens[b] + paths[b, j] to ctx_lens[b] + j, for every layer
 * and KV head of both pools (layout pool[block][layer][kv_head][slot][dim],
 * paged_kv_cache.cpp:13-21, 409-421).  Rows already in place are not touched.
 * A sequence whose path is malformed or reaches an unmapped page is left
 * unchanged and flagged (status[b] = 1).
 *
 *   new_ctx_lens [B] (optional): ctx_lens + L (or ctx_lens when rejected)
 *   status       [B] (optional): 0 committed, 1 rejected
 */
int cfa_kv_commit(void *k_pool, void *v_pool, const int32_t *block_tables,
                  int max_blocks_per_seq, const int32_t *ctx_lens, const int32_t *paths,
                  int path_stride, const int32_t *path_lens, int B, int num_blocks,
                  int num_layers, int n_kv_heads, int block_size, int head_dim, int elem_bytes,
                  int32_t *new_ctx_lens, int32_t *status, void *stream);

/* ---------------------------------------------------------------------------
 * W4A16 weight dequantisation.
 *
 * The reference's packed INT4 weights (dequantize.cuh:12-25): b_quant
 * [K/8, N] 32-bit words, nibble k % 8 of word (k/8, n) at bits 4*(k % 8),
 * unsigned; scales [K/group_size, N] fp16; zeros (optional) the same shape,
 * fp16.  out [K, N]: fp16 (out_bf16 = 0) w = (fp16(nibble) - z) * s in fp16
 * arithmetic, as int4_gemm_dequant.cu:20-31 (without zeros: fp16(nibble * s),
 * as int4_dequant_triton.py:74-78); bf16 (out_bf16 = 1) w = bf16((nibble - z)
 * * s) formed in fp32.  Feeds the GEMMs of int4_gemm_dequant_triton
 * (int4_dequant_triton.py:86-131) / launch_int4_gemm_dequant.
 */
int cfa_w4a16_dequant(const uint32_t *b_quant, const void *scales, const void *zeros, int K,
                      int N, int group_size, int out_bf16, void *out, void *stream);
/* As cfa_w4a16_dequant with the transposed output out [N, K] (K contiguous,
 * 16-byte aligned): the same values, in the layout the GEMM that follows
 * (x @ out^T) runs fastest on. */
int cfa_w4a16_dequant_t(const uint32_t *b_quant, const void *scales, const void *zeros, int K,
                        int N, int group_size, int out_bf16, void *out, void *stream);

/* Fused W4A16 GEMM: c [M, N] = a [M, K] x dequant(b_quant, scales) with the
 * dequantisation of cfa_w4a16_dequant (no zero points) done on the device
 * (in LDS for bf16 with M > 64, in registers otherwise) and fp32
 * accumulation on MFMA.  fp16 = 1: a and c fp16 (int4_gemm_dequant.cu /
 * int4_dequant_triton.py semantics); fp16 = 0: bf16.  N % 256 == 0 (bf16
 * with M > 64 and 16-byte aligned scales: N % 64 == 0), group_size % 64 == 0,
 * K % group_size == 0; a, b_quant, c 16-byte aligned, scales 8-byte
 * aligned. */
int cfa_w4a16_gemm(const void *a, const uint32_t *b_quant, const void *scales, int M, int N,
                   int K, int group_size, int fp16, void *c, void *stream);

/* Fused W4A16 GEMM with zero points, for many rows (the verify step's target
 * projections; replaces launch_int4_gemm_dequant / int4_gemm_dequant_triton,
 * int4_dequant_triton.py:86-131, for bf16 activations): c [M, N] bf16 =
 * a [M, K] bf16 x W with W = bf16((nibble - z) * s) exactly as
 * cfa_w4a16_dequant writes it (zeros may be NULL: z = 0), dequantised once
 * per 256 x 256 output tile into LDS, fp32 accumulation on MFMA.  N % 256 ==
 * 0, K % 32 == 0, group_size % 32 == 0 dividing K; a and c 16-byte aligned,
 * b_quant 4-byte, scales and zeros 2-byte.  Splits K over the work-groups
 * when the output tiles alone leave CUs idle: the fp32 partials go to
 * `workspace` (cfa_w4a16_gemm_zp_workspace_size bytes, 0 when no split is
 * used) and are summed in split order, so results are reproducible. */
size_t cfa_w4a16_gemm_zp_workspace_size(int M, int N, int K);
int cfa_w4a16_gemm_zp(const void *a, const uint32_t *b_quant, const void *scales,
                      const void *zeros, int M, int N, int K, int group_size, void *c,
                      void *workspace, size_t workspace_bytes, void *stream);
/* The same product with a SiLU-gated epilogue (the gate/up projection of a
 * Llama FFN; no counterpart in the reference, whose model runner is out of
 * this library's scope): the N columns of W hold, in each 64-column tile t,
 * gate columns for features 32t .. 32t + 31 followed by the up columns of the
 * same features; out [M, N / 2] = bf16(bf16(silu(g)) * u) with g and u the
 * product's columns rounded to bf16, bit-identical to cfa_w4a16_gemm_zp
 * followed by cfa_silu_mul on the de-interleaved [g | u] columns.  Shape
 * rules and workspace as cfa_w4a16_gemm_zp. */
int cfa_w4a16_gemm_zp_silu(const void *a, const uint32_t *b_quant, const void *scales,
                           const void *zeros, int M, int N, int K, int group_size, void *out,
                           void *workspace, size_t workspace_bytes, void *stream);
/* The same product left as its split-K fp32 partials (no counterpart in the
 * reference; for a consumer that sums them itself, cfa_rmsnorm_partials):
 * part [S, M, N] fp32 with S = cfa_w4a16_gemm_zp_splits(M, N, K) (>= 1; 0
 * for a shape the kernel does not take), slab s the product over split s's
 * k range, so that bf16 of their sum in slab order is cfa_w4a16_gemm_zp's
 * output.  part_bytes >= S * M * N * 4, 16-byte aligned. */
int cfa_w4a16_gemm_zp_splits(int M, int N, int K);
int cfa_w4a16_gemm_zp_partials(const void *a, const uint32_t *b_quant, const void *scales,
                               const void *zeros, int M, int N, int K, int group_size,
                               float *part, size_t part_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Fused layers of the model-scale verify step (bf16 activations, fp32 math;
 * no counterpart in the reference, whose model runner is out of this
 * library's scope).
 *
 * cfa_rmsnorm: h <- bf16(h + delta) when delta != NULL, then out <- bf16(h *
 *   rsqrt(mean(h^2) + eps) * weight); h, delta, out [M, d], weight [d];
 *   d % 8 == 0, 16-byte aligned rows.
 * cfa_rope_kv_paged / _strided: rotate-half rotary embedding (angle pos *
 *   theta^(-2i/D)) of the q and k heads of qkv [B*n, Hq + 2*Hkv, D]; writes
 *   q_out [B*n, Hq, D] and stores k (rotated) and v in the KV cache: paged
 *   pools [blocks][num_layers][Hkv][block_size][D] at slot base_lens[b] + j of
 *   `layer` (pages from block_tables [B, max_blocks]; an unmapped page is
 *   skipped); or strided caches at k_cache + b*ks[0] + h*ks[1] + slot*ks[2] +
 *   e*ks[3] (v likewise, with vs[3] == 1), slot = slots[b*n + j].
 *   positions [B*n].
 * cfa_silu_mul: out [M, F] = bf16(bf16(silu(g)) * u) for gu [M, 2F] = [g | u].
 */
int cfa_rmsnorm(void *h, const void *delta, const void *weight, void *out, int M, int d,
                float eps, void *stream);
/* The same with delta = bf16(sum of part[0 .. splits) in slab order), part
 * [splits, M, d] fp32 (the partials of cfa_w4a16_gemm_zp_partials): the bits
 * of cfa_w4a16_gemm_zp followed by cfa_rmsnorm, without the reduce pass. */
int cfa_rmsnorm_partials(void *h, const float *part, int splits, const void *weight, void *out,
                         int M, int d, float eps, void *stream);
int cfa_rope_kv_paged(const void *qkv, const int32_t *positions, int B, int n, int Hq, int Hkv,
                      int D, float theta, void *q_out, void *k_pool, void *v_pool, int layer,
                      int num_layers, int block_size, const int32_t *block_tables, int max_blocks,
                      const int32_t *base_lens, void *stream);
/* The same from the fused projection's split-K fp32 partials part [splits,
 * B*n, (Hq + 2*Hkv)*D] (cfa_w4a16_gemm_zp_partials): each element is bf16 of
 * their sum in slab order, the bits of cfa_w4a16_gemm_zp followed by
 * cfa_rope_kv_paged, without the reduce pass. */
int cfa_rope_kv_paged_partials(const float *part, int splits, const int32_t *positions, int B,
                               int n, int Hq, int Hkv, int D, float theta, void *q_out,
                               void *k_pool, void *v_pool, int layer, int num_layers,
                               int block_size, const int32_t *block_tables, int max_blocks,
                               const int32_t *base_lens, void *stream);
int cfa_rope_kv_strided(const void *qkv, const int32_t *positions, int B, int n, int Hq, int Hkv,
                        int D, float theta, void *q_out, void *k_cache, const int64_t *k_strides,
                        void *v_cache, const int64_t *v_strides, const int32_t *slots,
                        void *stream);
int cfa_silu_mul(const void *gu, void *out, int M, int F, void *stream);

/* Few-row bf16 GEMM: c [M, N] = a [M, K] x w [K, N], all row-major bf16, fp32
 * accumulation on MFMA, 1 <= M <= 128, N % 64 == 0, K % 128 == 0, pointers
 * 16-byte aligned.  Streams w once, split over `splits` equal k ranges
 * (0: the library's choice; otherwise a divisor of K / 128).  With more
 * than one split it needs `workspace` (cfa_gemm_bf16_skinny_workspace_size
 * bytes, 256-byte aligned) whose first 64 KiB are ZERO before its first
 * use: they hold per-tile arrival counters (N / 64 <= 16384) that every call
 * leaves at zero, so calls of any shape may share one workspace but must not
 * overlap.  Sums run in a fixed order (bitwise
 * reproducible).  Takes the place of the draft model's PyTorch GEMMs. */
size_t cfa_gemm_bf16_skinny_workspace_size(int M, int N, int K, int splits);
int cfa_gemm_bf16_skinny(const void *a, const void *w, void *c, int M, int N, int K, int splits,
                         void *workspace, size_t workspace_bytes, void *stream);
/* The same product with a SiLU-gated epilogue: w [K, N] holds, in each
 * 64-column tile t, gate columns for features 32t .. 32t + 31 followed by
 * the up columns of the same features; out [M, N / 2] = bf16(bf16(silu(g))
 * * u) with g and u the product's columns rounded to bf16, bit-identical to
 * cfa_gemm_bf16_skinny on the de-interleaved [g | u] weights followed by
 * cfa_silu_mul.  Workspace as cfa_gemm_bf16_skinny. */
int cfa_gemm_bf16_skinny_silu(const void *a, const void *w, void *out, int M, int N, int K,
                              int splits, void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Paged KV cache page tables (host metadata).
 *
 * Replaces the metadata half of PagedKVCache (paged_kv_cache.h:36-179,
 * paged_kv_cache.cpp:10-445; pybind names at pybind_module.cpp:20-99): page
 * reference counts and fill counts, the LIFO free list (the first page handed
 * out is page 0), prefix sharing of full prompt pages through chained block
 * hashes (paged_kv_cache.cpp:80-88), LRU retention and eviction of released
 * prefix pages, fork, and the per-batch staging of block tables and context
 * lengths for the kernels.  The K/V pools, the pinned host staging buffers and
 * the device block tables are the caller's: this library allocates no device
 * or pinned memory.  All calls on one cache are serialised by its lock.
 * Errors: CFA_ERR_STATE for an unknown sequence id (std::runtime_error in the
 * reference), CFA_ERR_RANGE for batch/table limits (std::out_of_range),
 * CFA_ERR_OUT_OF_PAGES when no page is free or evictable.
 */
typedef struct cfa_kv_cache cfa_kv_cache;

/* KVCacheConfig (paged_kv_cache.h:36-46), same fields and meaning. */
typedef struct cfa_kv_cache_config {
  uint32_t num_layers;
  uint32_t num_kv_heads;
  uint32_t head_dim;
  uint32_t block_size;
  uint64_t element_size_bytes;
  uint64_t total_gpu_blocks;
  uint32_t enable_prefix_caching; /* bool */
  uint32_t reserved;
  uint64_t max_supported_batch_size;
  uint64_t max_blocks_per_sequence;
} cfa_kv_cache_config;

/* KVCacheStats (paged_kv_cache.h:63-75), same fields and formulas
 * (paged_kv_cache.cpp:423-445). */
typedef struct cfa_kv_cache_stats {
  uint64_t total_blocks;
  uint64_t free_blocks;
  uint64_t allocated_blocks;
  uint64_t cached_prefix_blocks;
  uint64_t total_memory_bytes;
  uint64_t used_memory_bytes;
  double pool_utilization_ratio;
  uint32_t active_sequences_count;
  uint32_t reserved;
  uint64_t prefix_cache_hits;
  uint64_t prefix_cache_misses;
  uint64_t lru_evictions_count;
} cfa_kv_cache_stats;

/* PagedKVCache::PagedKVCache / ~PagedKVCache (paged_kv_cache.cpp:9-78),
 * metadata only. */
int cfa_kv_cache_create(const cfa_kv_cache_config *config, cfa_kv_cache **out);
void cfa_kv_cache_destroy(cfa_kv_cache *cache);

/* register_sequence_with_prefix (paged_kv_cache.cpp:167-253): reuses the
 * cached pages of the longest matching run of full prompt pages, allocates the
 * rest; *matched_tokens = tokens served from the prefix cache.  A sequence id
 * already registered is left as it is (matched 0). */
int cfa_kv_cache_register_sequence(cfa_kv_cache *cache, uint64_t sequence_id,
                                   const int32_t *prompt_tokens, int64_t n_tokens,
                                   uint32_t *matched_tokens);
/* append_tokens (paged_kv_cache.cpp:255-286). */
int cfa_kv_cache_append_tokens(cfa_kv_cache *cache, uint64_t sequence_id, uint32_t num_tokens);
/* unregister_sequence (paged_kv_cache.cpp:288-299); unknown ids are ignored. */
int cfa_kv_cache_unregister_sequence(cfa_kv_cache *cache, uint64_t sequence_id);
/* fork_sequence (paged_kv_cache.cpp:301-316).  An already registered child
 * releases its own pages first; parent == child is CFA_ERR_ARG.  Parent and
 * child share every page; the first append (or truncate) that would change a
 * shared, partly filled page gives the changing sequence a private copy and
 * queues the device copy of its slots (see cfa_kv_cache_pop_page_copies).
 * The reference shares the page for writing (paged_kv_cache.cpp:265-271). */
int cfa_kv_cache_fork_sequence(cfa_kv_cache *cache, uint64_t parent_sequence_id,
                               uint64_t child_sequence_id);
/* Rollback (no counterpart in the reference, which only grows sequences):
 * keep the first new_length tokens, release the pages past them (at least one
 * page stays).  Cutting inside a page that another sequence shares copies the
 * kept part to a private page (queued as for append); cutting inside a
 * private prefix page drops its prefix entry.  new_length above the current
 * length is CFA_ERR_ARG. */
int cfa_kv_cache_truncate_sequence(cfa_kv_cache *cache, uint64_t sequence_id, uint32_t new_length);
/* (pages - 1) * block_size + fill of the last page (paged_kv_cache.cpp:359-364). */
int cfa_kv_cache_context_length(cfa_kv_cache *cache, uint64_t sequence_id, uint32_t *length);
/* get_block_table (paged_kv_cache.cpp:398-407): *n_blocks = table length;
 * min(capacity, length) ids are copied to out (out may be NULL). */
int cfa_kv_cache_get_block_table(cfa_kv_cache *cache, uint64_t sequence_id, int32_t *out,
                                 int64_t capacity, int64_t *n_blocks);
/* prepare_batch_metadata (paged_kv_cache.cpp:318-396): writes the
 * [batch, max_blocks] block tables (-1 padded) and the context lengths into
 * the caller's host buffers (pinned for an asynchronous copy), then, when the
 * device buffers are given, enqueues both host-to-device copies on `stream`.
 * The host buffers must stay untouched until that copy has run.
 * *max_blocks_out = the batch's longest table (the descriptor's
 * max_blocks_per_seq).  Capacities are in int32 elements. */
int cfa_kv_cache_prepare_batch(cfa_kv_cache *cache, const uint64_t *sequence_ids, int batch_size,
                               int32_t *host_block_tables, int32_t *host_context_lens,
                               int64_t host_capacity, int32_t *dev_block_tables,
                               int32_t *dev_context_lens, int64_t dev_capacity,
                               int32_t *max_blocks_out, void *stream);
/* get_stats (paged_kv_cache.cpp:423-445). */
int cfa_kv_cache_get_stats(cfa_kv_cache *cache, cfa_kv_cache_stats *out);
/* Copy on write: a queued copy of slots [0, n_slots) of page src_block to
 * page dst_block, for every layer and KV head of both pools.  The caller runs
 * these copies (in order, before any write to dst_block) after each append or
 * truncate; no counterpart in the reference. */
typedef struct cfa_kv_page_copy {
  int32_t src_block;
  int32_t dst_block;
  int32_t n_slots;
} cfa_kv_page_copy;

/* Moves up to `capacity` queued copies, oldest first, into out and sets
 * *count to how many; with out == NULL or capacity <= 0 only reports the
 * number pending. */
int cfa_kv_cache_pop_page_copies(cfa_kv_cache *cache, cfa_kv_page_copy *out, int64_t capacity,
                                 int64_t *count);
/* Reference count, fill and LRU membership of one page (the reference's
 * PhysicalBlock fields, paged_kv_cache.h:48-55); for tests and monitoring. */
int cfa_kv_cache_block_info(cfa_kv_cache *cache, int32_t block_id, uint32_t *ref_count,
                            uint32_t *tokens_filled, int32_t *is_cached);

/* ---------------------------------------------------------------------------
 * Host uniform stream of the compatibility engine.
 *
 * The reference's SpeculativeEngine owns a std::mt19937 seeded with rng_seed
 * (speculative.h:83, speculative.cpp:8-9) and draws
 * std::uniform_real_distribution<float>(0, 1) once per acceptance test and once
 * per final draw (speculative.cpp:13-14, 64, 72).  These calls keep that
 * stream on the host so that SpeculativeEngine(config) produces the same
 * tokens as the reference for the same seed; the verification itself runs on
 * the GPU through cfa_chain_verify.
 */
typedef struct cfa_rng cfa_rng;

cfa_rng *cfa_rng_create(uint64_t seed);
void cfa_rng_destroy(cfa_rng *rng);
/* Copy the next n draws into out without consuming them. */
int cfa_rng_peek(const cfa_rng *rng, int n, float *out);
/* Consume n draws. */
int cfa_rng_advance(cfa_rng *rng, int n);

/* ---------------------------------------------------------------------------
 * Kernel timing (no counterpart in the reference; its speculative path only
 * reads host perf_counter around phases, cudaforge/speculative.py:107-147).
 *
 * When enabled, every kernel launch of this library is bracketed by two
 * hipEvents on the stream it runs on.  cfa_profile_query() synchronises on
 * the recorded events and returns the launch count and summed duration of one
 * kernel name (e.g. "chain_stats"); cfa_profile_reset() drops the records.
 */
int cfa_profile_enable(int on);
int cfa_profile_reset(void);
int cfa_profile_query(const char *kernel, int *count, double *total_ms);

#ifdef __cplusplus
}
#endif

#endif /* CUDAFORGE_AMD_H */
