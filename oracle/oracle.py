"""CPU oracle for the speculative-decoding verification path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this module, and only as the
checker / CPU baseline.  The product library (``cudaforge_amd``) never imports
it and fails loudly when its HIP library is missing.

Contents
  * ctypes bindings of ``spec_oracle.c`` (plain C restatement of
    ``csrc/src/scheduler/speculative.cpp:11-150`` and of the acceptance rules
    of ``cudaforge/speculative.py:57-211``; tree rejection sampling);
  * ctypes bindings of ``_ref/libref_spec.so`` -- the reference's own
    ``SpeculativeEngine`` compiled from its sources (only where the reference
    tree was mounted when ``make -C oracle`` ran);
  * torch-CPU restatements for tree attention over a paged KV cache (fp32
    masked SDPA; conventions of ``csrc/kernels/triton/flash_attn_triton.py:
    112-172``) and for the KV commit (``index_copy`` of accepted slots; page
    addressing of ``csrc/src/memory/paged_kv_cache.cpp:13-21,409-421``);
  * the context-length rule of ``paged_kv_cache.cpp:359-364``;
  * the sampler's keep rules and greedy top-k (``topk_keep``,
    ``sample_filtered``, ``topk_greedy``; ``sampling.h:61-186``).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

c_i32p = ctypes.POINTER(ctypes.c_int32)
c_f32p = ctypes.POINTER(ctypes.c_float)
c_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> None:
    """Compile the oracle (and oracle/_ref when the reference is mounted)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        # ORACLE_LIB_PATH: another build of spec_oracle.c (the sanitizer runs)
        path = os.environ.get("ORACLE_LIB_PATH") or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.orc_sample_from_distribution.restype = ctypes.c_int32
        L.orc_sample_from_distribution.argtypes = [c_f32p, ctypes.c_int64, ctypes.c_float]
        L.orc_sample_adjusted.restype = ctypes.c_int32
        L.orc_sample_adjusted.argtypes = [c_f32p, c_f32p, ctypes.c_int64, ctypes.c_float,
                                          ctypes.POINTER(ctypes.c_int)]
        L.orc_seq_sum.restype = ctypes.c_float
        L.orc_seq_sum.argtypes = [c_f32p, ctypes.c_int64]
        L.orc_argmax_first.restype = ctypes.c_int32
        L.orc_argmax_first.argtypes = [c_f32p, ctypes.c_int64]
        L.orc_chain_verify_batch.restype = ctypes.c_int
        L.orc_chain_verify_batch.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int64, c_f32p, c_f32p, c_i32p, c_f32p, ctypes.c_int32, ctypes.c_int,
            c_i32p, c_i32p, c_i32p, c_i32p, c_i32p]
        L.orc_softmax_rows.restype = None
        L.orc_softmax_rows.argtypes = [c_f32p, c_f32p, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_float]
        L.orc_verify_python.restype = ctypes.c_int
        L.orc_verify_python.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int64, c_f32p, c_f32p, c_i32p, c_f32p, ctypes.c_float,
            c_i32p, c_i32p, c_i32p]
        L.orc_py_sample_adjusted.restype = ctypes.c_int32
        L.orc_py_sample_adjusted.argtypes = [c_f32p, c_f32p, ctypes.c_int64, ctypes.c_float,
                                             ctypes.POINTER(ctypes.c_int)]
        L.orc_py_residual_weights.restype = ctypes.c_int
        L.orc_py_residual_weights.argtypes = [c_f32p, c_f32p, ctypes.c_int64, c_f32p]
        L.orc_py_bonus_weights.restype = None
        L.orc_py_bonus_weights.argtypes = [c_f32p, ctypes.c_int64, ctypes.c_float, c_f32p]
        L.orc_topp_keep.restype = None
        L.orc_topp_keep.argtypes = [c_f32p, ctypes.c_int64, ctypes.c_float, c_u8p]
        L.orc_sample_weights.restype = ctypes.c_int32
        L.orc_sample_weights.argtypes = [c_f32p, ctypes.c_int64, ctypes.c_float]
        L.orc_set_threads.restype = None
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_tree_verify.restype = ctypes.c_int
        L.orc_tree_verify.argtypes = [
            ctypes.c_int, ctypes.c_int64, ctypes.c_int64, c_i32p, c_i32p, c_f32p, c_f32p,
            ctypes.c_int32, c_f32p, ctypes.c_int, ctypes.c_int, c_i32p, c_i32p, c_i32p,
            c_i32p, c_i32p]
        _LIB = L
    return _LIB


def ref_lib() -> Optional[ctypes.CDLL]:
    """The reference's compiled SpeculativeEngine, or None if it was not built."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libref_spec.so")
        if not os.path.exists(path):
            return None
        L = ctypes.CDLL(path)
        L.ref_uniforms.restype = ctypes.c_int
        L.ref_uniforms.argtypes = [ctypes.c_uint64, ctypes.c_int, c_f32p]
        L.ref_verify.restype = ctypes.c_int
        L.ref_verify.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int64, c_i32p, c_f32p, c_f32p, ctypes.c_int32,
                                 c_i32p, c_i32p, c_i32p, c_i32p]
        _REF = L
    return _REF


def set_threads(n: int) -> None:
    """OpenMP threads of the batched oracle functions."""
    lib().orc_set_threads(int(n))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


# ---------------------------------------------------------------------------
# speculative.cpp restatement
# ---------------------------------------------------------------------------

def sample_from_distribution(probs, r: float) -> int:
    p = _f32(probs)
    return int(lib().orc_sample_from_distribution(_p(p, c_f32p), p.size, np.float32(r)))


def sample_adjusted(target_p, draft_q, r: float) -> tuple[int, bool]:
    t, d = _f32(target_p), _f32(draft_q)
    fb = ctypes.c_int(0)
    tok = lib().orc_sample_adjusted(_p(t, c_f32p), _p(d, c_f32p), t.size, np.float32(r),
                                    ctypes.byref(fb))
    return int(tok), bool(fb.value)


def seq_sum(x) -> float:
    a = _f32(x)
    return float(np.float32(lib().orc_seq_sum(_p(a, c_f32p), a.size)))


def argmax_first(x) -> int:
    a = _f32(x)
    return int(lib().orc_argmax_first(_p(a, c_f32p), a.size))


def chain_verify(tprobs, dprobs, tokens, uniforms, eos: int = -1, greedy: bool = False):
    """Batched cpp-mode chain verification (speculative.cpp:50-150 per row).

    tprobs [B,K+1,V], dprobs [B,K,V], tokens [B,K], uniforms [B,K+1].
    Returns dict of numpy arrays: accept_len [B], tokens [B,K+1] (accepted
    drafts then the final token, -1 padded), num_emitted [B], final [B], eos [B].
    """
    t, d = _f32(tprobs), _f32(dprobs)
    tok, U = _i32(tokens), _f32(uniforms)
    B, K1, V = t.shape
    K = K1 - 1
    assert d.shape == (B, K, V) and tok.shape == (B, K) and U.shape == (B, K + 1)
    out = dict(accept_len=np.zeros(B, np.int32), tokens=np.zeros((B, K + 1), np.int32),
               num_emitted=np.zeros(B, np.int32), final=np.zeros(B, np.int32),
               eos=np.zeros(B, np.int32))
    if K == 0:
        d = np.zeros((B, 1, V), np.float32)
    rc = lib().orc_chain_verify_batch(
        B, K, V, V, (K + 1) * V, max(K, 1) * V, _p(t, c_f32p), _p(d, c_f32p), _p(tok, c_i32p),
        _p(U, c_f32p), int(eos), int(bool(greedy)), _p(out["accept_len"], c_i32p),
        _p(out["tokens"], c_i32p), _p(out["num_emitted"], c_i32p), _p(out["final"], c_i32p),
        _p(out["eos"], c_i32p))
    if rc != 0:
        raise ValueError("chain_verify: token id out of range")
    return out


def softmax_rows(logits, temperature: float) -> np.ndarray:
    x = _f32(logits)
    V = x.shape[-1]
    rows = x.size // V
    p = np.empty_like(x)
    lib().orc_softmax_rows(_p(x, c_f32p), _p(p, c_f32p), rows, V, V, np.float32(temperature))
    return p


def python_verify(tprobs, dprobs, tokens, uniforms, top_p: float):
    """speculative.py:152-195 with fed uniforms [B, K+2] (columns 0..K-1 the
    acceptance draws, K the resample / bonus draw, K+1 the bonus after a
    rejection at the last position).  Returns (n, num_emitted, tokens [B,K+1]):
    n accepted drafts (batch-wide), num_emitted tokens per row (the
    reference's num_accepted), -1 padded tokens."""
    t, d = _f32(tprobs), _f32(dprobs)
    tok = _i32(tokens)
    U = _f32(uniforms)
    B, K1, V = t.shape
    K = K1 - 1
    assert U.shape == (B, K + 2), "python-mode uniforms are [B, K+2]"
    n = ctypes.c_int32(0)
    ne = ctypes.c_int32(0)
    out = np.zeros((B, K + 1), np.int32)
    if K == 0:
        d = np.zeros((B, 1, V), np.float32)
    rc = lib().orc_verify_python(B, K, V, V, (K + 1) * V, max(K, 1) * V, _p(t, c_f32p),
                                 _p(d, c_f32p), _p(tok, c_i32p), _p(U, c_f32p),
                                 np.float32(top_p), ctypes.byref(n), ctypes.byref(ne),
                                 _p(out, c_i32p))
    if rc != 0:
        raise ValueError("python_verify: token id out of range")
    return int(n.value), int(ne.value), out


def py_sample_adjusted(target_p, draft_q, u: float) -> tuple[int, bool]:
    """The python-mode residual draw (speculative.py:171-182)."""
    t, d = _f32(target_p), _f32(draft_q)
    fb = ctypes.c_int(0)
    tok = lib().orc_py_sample_adjusted(_p(t, c_f32p), _p(d, c_f32p), t.size, np.float32(u),
                                       ctypes.byref(fb))
    return int(tok), bool(fb.value)


def py_residual_weights(target_p, draft_q) -> tuple[np.ndarray, bool]:
    """The normalised weights the python-mode resample draws from
    (speculative.py:171-182) and whether the sum <= 1e-6 fallback applied."""
    t, d = _f32(target_p), _f32(draft_q)
    out = np.empty(t.size, np.float32)
    fb = lib().orc_py_residual_weights(_p(t, c_f32p), _p(d, c_f32p), t.size, _p(out, c_f32p))
    return out, bool(fb)


def py_bonus_weights(pk, top_p: float) -> np.ndarray:
    """The normalised weights the python-mode bonus draws from
    (speculative.py:57-84, :188-195)."""
    a = _f32(pk)
    out = np.empty(a.size, np.float32)
    lib().orc_py_bonus_weights(_p(a, c_f32p), a.size, np.float32(top_p), _p(out, c_f32p))
    return out


def topp_keep(p, top_p: float) -> np.ndarray:
    a = _f32(p)
    keep = np.zeros(a.size, np.uint8)
    lib().orc_topp_keep(_p(a, c_f32p), a.size, np.float32(top_p), _p(keep, c_u8p))
    return keep.astype(bool)


def topk_keep(p, top_k: int) -> np.ndarray:
    """Keep every p_i >= the top_k-th largest value (ties kept); top_k <= 0
    or >= V keeps everything.  No reference counterpart (the reference
    sampler takes top_k but never applies it, sampling.h:61-186)."""
    a = _f32(p).ravel()
    if top_k <= 0 or top_k >= a.size:
        return np.ones(a.size, bool)
    kth = np.sort(a)[::-1][top_k - 1]
    return a >= kth


def sample_filtered(p, r: float, top_p: float, top_k: int) -> int:
    """Keep rule (top-p of speculative.py:67-81 and top-k), renormalise by
    the sequential fp32 kept mass, python-mode inverse CDF (sample_weights)."""
    a = _f32(p).ravel()
    keep = topp_keep(a, top_p) & topk_keep(a, top_k)
    return sample_weights(np.where(keep, a, np.float32(0)).astype(np.float32), r)


def topk_greedy(rows, k: int) -> np.ndarray:
    """The k largest values of each row, largest first, equal values by lower
    index (sampling.h:107-135 for k = 1: the first argmax)."""
    x = np.asarray(rows, np.float32)
    out = np.empty((x.shape[0], k), np.int32)
    for r in range(x.shape[0]):
        order = np.lexsort((np.arange(x.shape[1]), -x[r].astype(np.float64)))
        out[r] = order[:k]
    return out


def sample_weights(w, r: float) -> int:
    """Python-mode draw from non-negative weights: normalise by the sequential
    fp32 sum, then the first index whose prefix sum exceeds r (never a
    zero-weight index; past the end of the sums, the last positive one)."""
    a = _f32(w)
    return int(lib().orc_sample_weights(_p(a, c_f32p), a.size, np.float32(r)))


def tree_verify(parent, tok, tprobs, dprobs, uniforms, eos: int = -1, greedy: bool = False):
    """Tree rejection sampling for one sequence.  Returns dict with path
    (accepted node ids starting at the root), final, eos, draws."""
    par, tk = _i32(parent), _i32(tok)
    t, d = _f32(tprobs), _f32(dprobs)
    U = _f32(uniforms)
    N, V = t.shape
    path = np.zeros(N, np.int32)
    plen, fin, ef, dr = (ctypes.c_int32(0) for _ in range(4))
    rc = lib().orc_tree_verify(N, V, V, _p(par, c_i32p), _p(tk, c_i32p), _p(t, c_f32p),
                               _p(d, c_f32p), int(eos), _p(U, c_f32p), U.size, int(bool(greedy)),
                               _p(path, c_i32p), ctypes.byref(plen), ctypes.byref(fin),
                               ctypes.byref(ef), ctypes.byref(dr))
    if rc != 0:
        raise ValueError("tree_verify: uniform stream too short")
    return dict(path=path[: plen.value].copy(), final=int(fin.value), eos=bool(ef.value),
                draws=int(dr.value))


# ---------------------------------------------------------------------------
# the reference's own engine (compiled from /root/reference when available)
# ---------------------------------------------------------------------------

def ref_uniforms(seed: int, n: int) -> np.ndarray:
    L = ref_lib()
    assert L is not None, "oracle/_ref not built"
    out = np.zeros(n, np.float32)
    L.ref_uniforms(seed, n, _p(out, c_f32p))
    return out


def ref_verify(seed: int, tokens, dprobs, tprobs, eos: int, greedy: bool = False):
    """Successive verify_candidates(_greedy) calls on one reference engine.

    tokens [C,K], dprobs [C,K,V], tprobs [C,K+1,V].  Returns dict of arrays
    (accepted [C,K] -1 padded, num_accepted [C], final [C], eos [C]) or raises
    ValueError where the reference threw std::invalid_argument."""
    L = ref_lib()
    assert L is not None, "oracle/_ref not built"
    tok = _i32(tokens)
    d, t = _f32(dprobs), _f32(tprobs)
    C, K = tok.shape
    V = t.shape[-1]
    acc = np.zeros((C, K), np.int32)
    na, fin, ef = (np.zeros(C, np.int32) for _ in range(3))
    if d.size == 0:
        d = np.zeros((C, max(K, 1), V), np.float32)
    rc = L.ref_verify(seed, int(bool(greedy)), C, K, V, _p(tok, c_i32p), _p(d, c_f32p),
                      _p(t, c_f32p), int(eos), _p(acc, c_i32p), _p(na, c_i32p),
                      _p(fin, c_i32p), _p(ef, c_i32p))
    if rc != 0:
        raise ValueError("Incompatible draft and target tensor dimensions in SpeculativeEngine.")
    return dict(accepted=acc, num_accepted=na, final=fin, eos=ef)


# ---------------------------------------------------------------------------
# tree attention / KV commit / page metadata (torch-CPU, fp32)
# ---------------------------------------------------------------------------

def binary_tree_parents(n_nodes: int) -> np.ndarray:
    """BFS-numbered complete binary tree: parent(i) = (i-1)>>1, parent(0) = -1."""
    p = (np.arange(n_nodes) - 1) >> 1
    p[0] = -1
    return p.astype(np.int32)


def ancestor_masks(parent: Sequence[int]) -> np.ndarray:
    """uint64 per node: bit j set iff j is an ancestor of i or i itself."""
    n = len(parent)
    assert n <= 64
    m = np.zeros(n, np.uint64)
    for i in range(n):
        bits = np.uint64(1) << np.uint64(i)
        if parent[i] >= 0:
            bits |= m[parent[i]]
        m[i] = bits
    return m


def context_length(num_blocks: int, block_size: int, last_block_filled: int) -> int:
    """paged_kv_cache.cpp:359-364: (blocks - 1) * block_size + last filled."""
    return (num_blocks - 1) * block_size + last_block_filled


def gather_pages(pool, block_table, n_tokens: int, layer: int, block_size: int):
    """Gather [n_tokens, Hkv, D] rows of one layer from a pool laid out as
    [num_blocks, num_layers, Hkv, block_size, D] (paged_kv_cache.cpp:13-21,
    409-421: block_id * bytes_per_block + layer * layer_block_bytes)."""
    import torch

    pos = torch.arange(n_tokens)
    blk = torch.as_tensor(block_table, dtype=torch.long)[pos // block_size]
    off = pos % block_size
    # pool[blk, layer, :, off, :] -> [n, Hkv, D]
    return pool[blk, layer][torch.arange(n_tokens), :, off, :]


def tree_attention(q, k_pool, v_pool, block_tables, ctx_lens, layer: int, tree_mask,
                   block_size: int, sm_scale: float):
    """fp32 masked SDPA.  q [B,N,Hq,D]; the tree's own K/V live in the pool at
    positions ctx_len + node; query i sees positions [0, ctx_len) and tree
    positions of its ancestors-or-self.  Returns [B,N,Hq,D] fp32."""
    import torch

    B, N, Hq, D = q.shape
    Hkv = k_pool.shape[2]
    g = Hq // Hkv
    out = torch.empty(B, N, Hq, D, dtype=torch.float32)
    tm = np.asarray(tree_mask, dtype=np.uint64)
    allow_tree = torch.tensor([[bool((int(tm[i]) >> j) & 1) for j in range(N)] for i in range(N)])
    for b in range(B):
        L = int(ctx_lens[b])
        k = gather_pages(k_pool, block_tables[b], L + N, layer, block_size).float()
        v = gather_pages(v_pool, block_tables[b], L + N, layer, block_size).float()
        mask = torch.ones(N, L + N, dtype=torch.bool)
        mask[:, L:] = allow_tree
        for h in range(Hq):
            kh = k[:, h // g, :]
            vh = v[:, h // g, :]
            s = (q[b, :, h, :].float() @ kh.T) * sm_scale
            s = s.masked_fill(~mask, float("-inf"))
            out[b, :, h, :] = torch.softmax(s, dim=-1) @ vh
    return out


def kv_commit(k_pool, v_pool, block_tables, ctx_lens, paths, path_lens, block_size: int):
    """Move the accepted tree nodes' K/V (slot ctx_len + node) to positions
    ctx_len + j, for every layer and head.  paths [B, Lmax] node ids with the
    root (node 0) first; path_lens [B].  Returns new (k_pool, v_pool)
    (copies) and the committed context lengths ctx_len + path_len."""
    import torch

    k2, v2 = k_pool.clone(), v_pool.clone()
    new_lens = []
    for b in range(len(ctx_lens)):
        L = int(ctx_lens[b])
        n = int(path_lens[b])
        bt = torch.as_tensor(block_tables[b], dtype=torch.long)
        src = torch.tensor([L + int(paths[b][j]) for j in range(n)], dtype=torch.long)
        dst = torch.arange(L, L + n)
        # read all sources first (index_copy semantics), then write
        ks = k_pool[bt[src // block_size], :, :, src % block_size, :].clone()
        vs = v_pool[bt[src // block_size], :, :, src % block_size, :].clone()
        k2[bt[dst // block_size], :, :, dst % block_size, :] = ks
        v2[bt[dst // block_size], :, :, dst % block_size, :] = vs
        new_lens.append(L + n)
    return k2, v2, np.asarray(new_lens, np.int32)
