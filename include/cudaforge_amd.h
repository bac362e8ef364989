/*
 * cudaforge_amd.h -- C ABI of the MI355X (gfx950) speculative-decoding
 * verification library (libcfa.so).
 *
 * Every entry point takes plain pointers and sizes.  Pointers named as device
 * buffers are HIP device addresses (e.g. torch.Tensor.data_ptr()); `stream` is
 * a hipStream_t (NULL = default stream) and all device work is enqueued on it
 * in order, without host synchronisation.  The library allocates no device
 * memory: scratch space is the caller's `workspace`.
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

/* input_kind */
#define CFA_INPUT_PROBS 0  /* rows are probabilities (the C++ engine's input) */
#define CFA_INPUT_LOGITS 1 /* rows are logits; softmax(logits / T) is fused */

/* mode */
#define CFA_MODE_CPP 0    /* per-row rules of speculative.cpp:50-103 */
#define CFA_MODE_PYTHON 1 /* batch lock-step rules of speculative.py:152-195 */
#define CFA_MODE_GREEDY 2 /* speculative.cpp:105-150 */

/* Message of this thread's last failed call ("" if none). */
const char *cfa_last_error(void);

/* Library ABI version (major * 100 + minor). */
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
 *   uniforms [B, K+1] fp32 in [0, 1):
 *     CFA_MODE_CPP: the draws the reference takes from its mt19937, in order
 *       (one per acceptance test, then one for the resample / bonus draw);
 *     CFA_MODE_PYTHON: columns 0..K-1 replace torch.rand_like at
 *       speculative.py:161, column K drives the resample / bonus draw.
 *   top_p    nucleus threshold of the python-mode bonus draw (speculative.py:67-81)
 *   eos_token_id  (< 0: none) CFA_MODE_CPP / GREEDY only
 *
 * Outputs (device, int32):
 *   out_accept_len  [B]    accepted draft tokens (the reference's num_accepted;
 *                          python mode: the batch-wide count n, speculative.py:166)
 *   out_tokens      [B, K+1] accepted drafts then the final token, -1 padded
 *   out_num_emitted [B]    valid entries of out_tokens
 *   out_final       [B]    final_token (resample or bonus draw)
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
 *   q        [B, N, n_q_heads, 128] bf16 -- queries of the N draft-tree nodes
 *   block_tables [B, max_blocks_per_seq] int32, ctx_lens [B] int32
 *   the tree's own K/V sit at positions ctx_len .. ctx_len + N - 1
 *   tree_mask  uint64 per node (bit j: node j is an ancestor of, or is, the
 *              node), [N] shared (stride 0) or [B, N] (stride N)
 *   max_keys   host-side bound on ctx_len + N over the batch (plans the splits)
 *   num_splits key-range splits (0: automatic); splits > 1 need workspace
 *   out        [B, N, n_q_heads, 128] bf16
 * Query (node i, head hq) attends to context positions [0, ctx_len) and to
 * tree positions ctx_len + j with bit j of tree_mask[i]; scores scale by
 * sm_scale; fp32 softmax and accumulation.
 */
size_t cfa_tree_attention_workspace_size(int B, int N, int n_q_heads, int n_kv_heads,
                                         int head_dim, int max_keys, int num_splits);

int cfa_tree_attention(const void *q, const void *k_pool, const void *v_pool,
                       const int32_t *block_tables, int max_blocks_per_seq,
                       const int32_t *ctx_lens, int num_blocks, int num_layers, int layer,
                       int block_size, const uint64_t *tree_mask, int64_t tree_mask_stride_b,
                       int B, int N, int n_q_heads, int n_kv_heads, int head_dim,
                       float sm_scale, int max_keys, int num_splits, void *out,
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
 * (optional; 1 when the uniform stream ran out).  out_target_probs /
 * out_draft_probs (optional, [B, N, V]) receive the probabilities of the rows
 * the walk visited.
 */
int cfa_tree_verify(const float *target, int64_t t_stride_b, int64_t t_stride_n,
                    const float *draft, int64_t d_stride_b, int64_t d_stride_n, int input_kind,
                    const int32_t *parents, int64_t parents_stride_b, const int32_t *node_tokens,
                    const float *uniforms, int n_uniforms, int B, int N, int V,
                    float temperature, int mode, int32_t eos_token_id, int32_t *out_path,
                    int32_t *out_path_len, int32_t *out_tokens, int32_t *out_num_emitted,
                    int32_t *out_final, int32_t *out_eos, int32_t *out_status,
                    float *out_target_probs, float *out_draft_probs, void *stream);

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
