"""One speculative verify step at model scale: a draft proposes a token tree,
the target scores it, and the tree is verified and committed.

This is the end-to-end shape of the reference's speculative loop
(``cudaforge/speculative.py:99-217``: draft proposal, one target forward over
the candidates, acceptance, bonus token) with a draft-token tree in place of
the chain, as a random-initialised Llama-3-8B-shape target with W4A16 weights
and a 1B-shape bf16 draft.  The verification path runs on this library's
kernels:

* tree expansion    ``cfa_sample`` (children drawn i.i.d. from the draft
                    softmax, or greedy top-2);
* tree attention    ``cfa_tree_attention`` over the target's paged KV pools;
* verification      ``cfa_tree_verify`` (multi-candidate rejection sampling,
                    longest accepted path, bonus token);
* KV commit         ``cfa_kv_commit`` plus the page-table rollback of
                    ``PagedKVCache.truncate_sequence``;
* W4A16 weights     ``cfa_w4a16_dequant_t`` (the reference's packed INT4
                    format, ``int4_gemm_dequant.cu:20-31``, dequantised as
                    [N, K]) feeding PyTorch-ROCm GEMMs;
* fused layers      ``cfa_rmsnorm`` (with the residual add),
                    ``cfa_rope_kv_paged`` (rotary embedding plus the KV-cache
                    write), ``cfa_silu_mul``;
* draft projections ``cfa_gemm_bf16_skinny`` (few-row split-K GEMM that
                    streams the weights once) for levels of <= 128 rows.

The draft keeps its own paged pools (head_dim 64, each sequence's pages
contiguous) and attends with the same tree-attention kernel, one tree level
at a time (``first_node``); its accepted nodes move with ``cfa_kv_commit``.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from . import _lib
from . import tree as T
from .kv_cache import KVCacheConfig, PagedKVCache
from .sampling import expand_tree_level
from .verify import (_stream_ptr, check_status, kv_commit, tree_attention,
                     tree_attention_workspace_bytes, tree_verify)
from .w4a16 import W4A16Linear

__all__ = ["LlamaShape", "TARGET_8B", "DRAFT_1B", "TargetModel", "DraftModel", "TreeSpeculator",
           "StepResult"]


@dataclass(frozen=True)
class LlamaShape:
    n_layers: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    rope_theta: float = 500000.0
    eps: float = 1e-5


TARGET_8B = LlamaShape(32, 4096, 32, 8, 128, 14336, 128256)
DRAFT_1B = LlamaShape(16, 2048, 32, 8, 64, 8192, 128256)


# ---------------------------------------------------------------------------
# shared pieces
# ---------------------------------------------------------------------------

def rmsnorm_(h: torch.Tensor, delta: Optional[torch.Tensor], w: torch.Tensor, eps: float,
             out: torch.Tensor) -> torch.Tensor:
    """h += delta (bf16, in place) when delta is given; out = RMSNorm(h) * w
    (cfa_rmsnorm)."""
    M, d = h.shape
    rc = _lib.load().cfa_rmsnorm(h.data_ptr(), delta.data_ptr() if delta is not None else None,
                                 w.data_ptr(), out.data_ptr(), M, d, float(eps),
                                 _stream_ptr(h.device))
    _lib.check(rc, "cfa_rmsnorm")
    return out


def add_norm_(h: torch.Tensor, delta: Optional[torch.Tensor], w: torch.Tensor, eps: float,
              out: torch.Tensor) -> torch.Tensor:
    """rmsnorm_ with delta given as bf16 [M, d], as fp32 split-K partials
    [S, M, d] of the W4A16 GEMM (summed in slab order, rounded to bf16, then
    added: cfa_rmsnorm_partials), or None."""
    if delta is None or delta.dim() == 2:
        return rmsnorm_(h, delta, w, eps, out)
    S, M, d = delta.shape
    if h.shape != (M, d) or delta.dtype != torch.float32 or not delta.is_contiguous():
        raise ValueError("partials must be contiguous fp32 [S, M, d]")
    rc = _lib.load().cfa_rmsnorm_partials(h.data_ptr(), delta.data_ptr(), S, w.data_ptr(),
                                          out.data_ptr(), M, d, float(eps), _stream_ptr(h.device))
    _lib.check(rc, "cfa_rmsnorm_partials")
    return out


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """[M, 2F] = [g | u] -> silu(g) * u in bf16 (cfa_silu_mul)."""
    M, F2 = gu.shape
    out = torch.empty(M, F2 // 2, dtype=gu.dtype, device=gu.device)
    rc = _lib.load().cfa_silu_mul(gu.data_ptr(), out.data_ptr(), M, F2 // 2, _stream_ptr(gu.device))
    _lib.check(rc, "cfa_silu_mul")
    return out


def skinny_gemm_workspace_bytes(M: int, N: int, K: int, splits: int = 0) -> int:
    """Bytes of workspace cfa_gemm_bf16_skinny needs (0: none)."""
    return int(_lib.load().cfa_gemm_bf16_skinny_workspace_size(M, N, K, splits))


def skinny_gemm(a: torch.Tensor, w: torch.Tensor, workspace: Optional[torch.Tensor] = None, *,
                splits: int = 0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """a [M, K] @ w [K, N] in bf16 for M <= 128 (cfa_gemm_bf16_skinny).
    `workspace` must have been zeroed before its first use and is left
    reusable; calls sharing it must not overlap."""
    M, K = a.shape
    N = w.shape[1]
    if w.shape[0] != K:
        raise ValueError("inner dimensions differ")
    if a.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("a and w must be bfloat16")
    if not (a.is_contiguous() and w.is_contiguous()):
        raise ValueError("a and w must be contiguous (row-major)")
    if out is None:
        out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    ws_ptr, ws_n = (workspace.data_ptr(), workspace.numel() * workspace.element_size()) \
        if workspace is not None else (None, 0)
    rc = _lib.load().cfa_gemm_bf16_skinny(a.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K,
                                          splits, ws_ptr, ws_n, _stream_ptr(a.device))
    _lib.check(rc, "cfa_gemm_bf16_skinny")
    return out


def interleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    """[K, 2F] = [gate | up] -> the layout cfa_gemm_bf16_skinny_silu takes:
    64-column tile t = gate features 32t .. 32t + 31, then their up columns."""
    K, F2 = w.shape
    F = F2 // 2
    if F % 32:
        raise ValueError("F must be a multiple of 32")
    return torch.stack([w[:, :F].reshape(K, F // 32, 32), w[:, F:].reshape(K, F // 32, 32)],
                       dim=2).reshape(K, F2).contiguous()


def deinterleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    """Inverse of interleave_gate_up (columns of a [.., 2F] tensor)."""
    lead, F2 = w.shape[:-1], w.shape[-1]
    v = w.reshape(*lead, F2 // 64, 2, 32)
    return torch.cat([v[..., 0, :].reshape(*lead, F2 // 2), v[..., 1, :].reshape(*lead, F2 // 2)],
                     dim=-1)


def skinny_gemm_silu(a: torch.Tensor, w_il: torch.Tensor, workspace: Optional[torch.Tensor] = None,
                     *, splits: int = 0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(a @ W_gate) * (a @ W_up) for M <= 128 with the gate/up weights in
    the interleave_gate_up layout (cfa_gemm_bf16_skinny_silu): bit-identical
    to silu_mul(skinny_gemm(a, W)) on the [gate | up] weights."""
    M, K = a.shape
    N = w_il.shape[1]
    if w_il.shape[0] != K:
        raise ValueError("inner dimensions differ")
    if a.dtype != torch.bfloat16 or w_il.dtype != torch.bfloat16:
        raise ValueError("a and w must be bfloat16")
    if not (a.is_contiguous() and w_il.is_contiguous()):
        raise ValueError("a and w must be contiguous (row-major)")
    if out is None:
        out = torch.empty(M, N // 2, dtype=a.dtype, device=a.device)
    ws_ptr, ws_n = (workspace.data_ptr(), workspace.numel() * workspace.element_size()) \
        if workspace is not None else (None, 0)
    rc = _lib.load().cfa_gemm_bf16_skinny_silu(a.data_ptr(), w_il.data_ptr(), out.data_ptr(), M,
                                               N, K, splits, ws_ptr, ws_n, _stream_ptr(a.device))
    _lib.check(rc, "cfa_gemm_bf16_skinny_silu")
    return out


def rope_kv_pools(qkv: torch.Tensor, pos: torch.Tensor, B: int, n: int, s: "LlamaShape",
                  q_out: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, layer: int,
                  block_tables: torch.Tensor, base: torch.Tensor) -> None:
    """Rotary embedding of q and k from qkv [B*n, (Hq+2Hkv)*D]; q -> q_out,
    k and v -> slots base + j of `layer` in the paged pools
    [blocks, layers, Hkv, block_size, D].  qkv may also be the W4A16 GEMM's
    fp32 split-K partials [S, B*n, (Hq+2Hkv)*D], summed in slab order and
    rounded to bf16 element by element (cfa_rope_kv_paged_partials)."""
    if qkv.dim() == 3:
        if qkv.dtype != torch.float32 or not qkv.is_contiguous():
            raise ValueError("partials must be contiguous fp32 [S, M, N]")
        rc = _lib.load().cfa_rope_kv_paged_partials(
            qkv.data_ptr(), qkv.shape[0], pos.data_ptr(), B, n, s.n_heads, s.n_kv_heads,
            s.head_dim, float(s.rope_theta), q_out.data_ptr(), k_pool.data_ptr(),
            v_pool.data_ptr(), layer, k_pool.shape[1], k_pool.shape[3], block_tables.data_ptr(),
            block_tables.shape[1], base.data_ptr(), _stream_ptr(qkv.device))
        _lib.check(rc, "cfa_rope_kv_paged_partials")
        return
    rc = _lib.load().cfa_rope_kv_paged(
        qkv.data_ptr(), pos.data_ptr(), B, n, s.n_heads, s.n_kv_heads, s.head_dim,
        float(s.rope_theta), q_out.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
        layer, k_pool.shape[1], k_pool.shape[3], block_tables.data_ptr(), block_tables.shape[1],
        base.data_ptr(), _stream_ptr(qkv.device))
    _lib.check(rc, "cfa_rope_kv_paged")


def rope_kv_paged(qkv: torch.Tensor, pos: torch.Tensor, B: int, n: int, s: "LlamaShape",
                  q_out: torch.Tensor, kv: PagedKVCache, layer: int, block_tables: torch.Tensor,
                  base: torch.Tensor) -> None:
    """rope_kv_pools into a PagedKVCache's pools."""
    rope_kv_pools(qkv, pos, B, n, s, q_out, kv.key_pool, kv.value_pool, layer, block_tables, base)


def rope_kv_strided(qkv: torch.Tensor, pos: torch.Tensor, B: int, n: int, s: "LlamaShape",
                    q_out: torch.Tensor, kT: torch.Tensor, v: torch.Tensor,
                    slots: torch.Tensor) -> None:
    """As rope_kv_paged into a contiguous cache: kT [B, Hkv, D, S] (K stored
    transposed), v [B, Hkv, S, D], slot of token (b, j) = slots[b, j]."""
    ks = (ctypes.c_int64 * 4)(kT.stride(0), kT.stride(1), kT.stride(3), kT.stride(2))
    vs = (ctypes.c_int64 * 4)(v.stride(0), v.stride(1), v.stride(2), v.stride(3))
    rc = _lib.load().cfa_rope_kv_strided(
        qkv.data_ptr(), pos.data_ptr(), B, n, s.n_heads, s.n_kv_heads, s.head_dim,
        float(s.rope_theta), q_out.data_ptr(), kT.data_ptr(), ks, v.data_ptr(), vs,
        slots.data_ptr(), _stream_ptr(qkv.device))
    _lib.check(rc, "cfa_rope_kv_strided")


def _randn(shape, gen, device, scale=1.0, dtype=torch.bfloat16):
    return (scale * torch.randn(shape, device=device, generator=gen)).to(dtype)


# ---------------------------------------------------------------------------
# target: W4A16 Llama shape over the paged cache, tree attention kernel
# ---------------------------------------------------------------------------

class TargetModel:
    def __init__(self, shape: LlamaShape, device, seed: int = 0, group: int = 128):
        if shape.head_dim != 128:
            raise ValueError("the tree-attention kernel takes head_dim 128")
        s = self.shape = shape
        g = torch.Generator(device=device).manual_seed(seed)
        d, hd = s.d_model, s.head_dim
        qkv_n = (s.n_heads + 2 * s.n_kv_heads) * hd
        self.embed = _randn((s.vocab, d), g, device)
        self.layers = []
        for _ in range(s.n_layers):
            self.layers.append(dict(
                attn_norm=torch.ones(d, dtype=torch.bfloat16, device=device),
                wqkv=W4A16Linear(d, qkv_n, device, g, group),
                wo=W4A16Linear(s.n_heads * hd, d, device, g, group),
                ffn_norm=torch.ones(d, dtype=torch.bfloat16, device=device),
                # gate/up in the interleaved layout of the SiLU-gated
                # epilogue (interleave_gate_up; random weights, so drawn in
                # that layout directly)
                wgu=W4A16Linear(d, 2 * s.ffn, device, g, group),
                wdown=W4A16Linear(s.ffn, d, device, g, group)))
        self.norm = torch.ones(d, dtype=torch.bfloat16, device=device)
        # stored [V, d] and used through its transposed view: at M = 504 rows,
        # d = 4096, V = 128256 hipBLASLt runs x @ W^T in ~575 us against
        # ~603 us for x @ W with W [d, V] (the draft's small-M head is the
        # other way round and stays [d, V])
        self.lm_head = _randn((s.vocab, d), g, device, 1.0 / math.sqrt(d)).t()
        biggest = max(d * qkv_n, s.n_heads * hd * d, d * 2 * s.ffn, s.ffn * d)
        self.scratch = torch.empty(biggest, dtype=torch.bfloat16, device=device)
        self.attn_ws = None

    def forward_tree(self, tokens: torch.Tensor, positions: torch.Tensor, kv: PagedKVCache,
                     block_tables: torch.Tensor, base_lens: torch.Tensor, masks: torch.Tensor,
                     max_keys: int) -> torch.Tensor:
        """tokens / positions [B, N]; the nodes' K/V go to slots base + node
        of every layer; returns fp32 logits [B, N, V]."""
        s = self.shape
        B, N = tokens.shape
        hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
        need = tree_attention_workspace_bytes(B, N, Hq, Hkv, hd, max_keys)
        if self.attn_ws is None or self.attn_ws.numel() < need:
            self.attn_ws = torch.empty(max(need, 1), dtype=torch.uint8, device=tokens.device)
        M = B * N
        pos = positions.reshape(-1).to(torch.int32).contiguous()
        base_i = base_lens.to(torch.int32).contiguous()
        h = self.embed[tokens.reshape(-1).long()]               # [B*N, d], a copy
        x = torch.empty_like(h)
        q = torch.empty(B, N, Hq, hd, dtype=torch.bfloat16, device=tokens.device)
        delta = None
        # the QKV, O and down projections hand their split-K partials (in
        # self.scratch) straight to their consumers -- the rope / K-V write
        # and the residual add + RMSNorm (add_norm_) -- which sum them before
        # the next GEMM reuses the scratch
        for li, L in enumerate(self.layers):
            add_norm_(h, delta, L["attn_norm"], s.eps, x)        # h += delta; x = norm(h)
            qkv = L["wqkv"].partials(x, self.scratch)            # summed by the rope kernel
            rope_kv_paged(qkv, pos, B, N, s, q, kv, li, block_tables, base_i)
            o = tree_attention(q, kv.key_pool, kv.value_pool, block_tables, base_lens, masks,
                               layer=li, max_keys=max_keys, workspace=self.attn_ws)
            add_norm_(h, L["wo"].partials(o.reshape(M, Hq * hd), self.scratch), L["ffn_norm"],
                      s.eps, x)
            a = L["wgu"].silu_gated(x, self.scratch)
            delta = L["wdown"].partials(a, self.scratch)
        add_norm_(h, delta, self.norm, s.eps, x)
        return (x @ self.lm_head).float().view(B, N, s.vocab)


# ---------------------------------------------------------------------------
# draft: bf16 Llama shape, its own paged pools, the tree-attention kernel
# ---------------------------------------------------------------------------

class DraftModel:
    """A bf16 Llama-shape drafter.  Its KV cache is a pair of paged pools
    [B * pages, layers, Hkv, 16, head_dim] whose block table gives sequence b
    the pages b * pages .. (b + 1) * pages - 1, so a tree level attends
    through ``cfa_tree_attention`` (queries: the level's nodes) and accepted
    nodes move with ``cfa_kv_commit``, exactly as in the target's cache."""

    block_size = 16

    def __init__(self, shape: LlamaShape, device, B: int, max_slots: int, seed: int = 1):
        s = self.shape = shape
        g = torch.Generator(device=device).manual_seed(seed)
        d, hd = s.d_model, s.head_dim
        qkv_n = (s.n_heads + 2 * s.n_kv_heads) * hd
        self.embed = _randn((s.vocab, d), g, device)
        self.layers = []
        for _ in range(s.n_layers):
            self.layers.append(dict(
                attn_norm=torch.ones(d, dtype=torch.bfloat16, device=device),
                wqkv=_randn((d, qkv_n), g, device, 1.0 / math.sqrt(d)),
                wo=_randn((s.n_heads * hd, d), g, device, 1.0 / math.sqrt(s.n_heads * hd)),
                ffn_norm=torch.ones(d, dtype=torch.bfloat16, device=device),
                # gate/up in the interleave_gate_up layout (the fused
                # SiLU-gated projection's)
                wgu=interleave_gate_up(_randn((d, 2 * s.ffn), g, device, 1.0 / math.sqrt(d))),
                wdown=_randn((s.ffn, d), g, device, 1.0 / math.sqrt(s.ffn))))
        self.norm = torch.ones(d, dtype=torch.bfloat16, device=device)
        self.lm_head = self.embed.t().contiguous()              # tied embeddings
        bs = self.block_size
        pages = (max_slots + bs - 1) // bs
        self.B, self.pages = B, pages
        self.max_slots = pages * bs
        self.k_pool = torch.zeros(B * pages, s.n_layers, s.n_kv_heads, bs, hd,
                                  dtype=torch.bfloat16, device=device)
        self.v_pool = torch.zeros_like(self.k_pool)
        self.block_tables = torch.arange(B * pages, dtype=torch.int32,
                                         device=device).view(B, pages).contiguous()
        # one workspace for every level, sized for the most query rows a call
        # takes: captured graphs keep using it
        max_q = min(64, 256 // (s.n_heads // s.n_kv_heads))
        need = tree_attention_workspace_bytes(B, max_q, s.n_heads, s.n_kv_heads, hd, self.max_slots)
        self.attn_ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
        # the projections of levels with B * n <= 128 rows run on
        # cfa_gemm_bf16_skinny; one zeroed workspace serves all of them
        gemm_need = max(skinny_gemm_workspace_bytes(128, w.shape[1], w.shape[0])
                        for w in self.layers[0].values() if w.dim() == 2)
        self.gemm_ws = torch.zeros(max(gemm_need, 65536), dtype=torch.uint8, device=device)

    def _mm(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        if x.shape[0] <= 128:
            return skinny_gemm(x, w, self.gemm_ws)
        return x @ w

    def _ffn_up(self, x: torch.Tensor, w_il: torch.Tensor) -> torch.Tensor:
        """silu(x @ W_gate) * (x @ W_up), W in the interleave_gate_up layout."""
        if x.shape[0] <= 128:
            return skinny_gemm_silu(x, w_il, self.gemm_ws)
        return silu_mul(deinterleave_gate_up(x @ w_il).contiguous())

    def forward_level(self, tokens: torch.Tensor, positions: torch.Tensor, base: torch.Tensor,
                      lo: int, masks: torch.Tensor) -> torch.Tensor:
        """Tree nodes lo .. lo + n - 1 (tokens / positions [B, n]; their K/V go
        to slots base + node) attend to the context [0, base) and to their
        ancestors among nodes 0 .. lo + n - 1 (masks: the tree's ancestor
        masks, int64 [N]).  Returns fp32 logits [B, n, V]."""
        s = self.shape
        B, n = tokens.shape
        hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
        dev = tokens.device
        hi = lo + n
        pos = positions.reshape(-1).to(torch.int32).contiguous()
        base_i = base.to(torch.int32).contiguous()
        slot0 = (base_i + lo).contiguous()                      # slot of node lo
        lvl_masks = masks[:hi].contiguous()
        h = self.embed[tokens.reshape(-1).long()]
        x = torch.empty_like(h)
        q = torch.empty(B, n, Hq, hd, dtype=torch.bfloat16, device=dev)
        delta = None
        for li, L in enumerate(self.layers):
            rmsnorm_(h, delta, L["attn_norm"], s.eps, x)
            qkv = self._mm(x, L["wqkv"])
            rope_kv_pools(qkv, pos, B, n, s, q, self.k_pool, self.v_pool, li, self.block_tables,
                          slot0)
            # max_keys is the cache capacity: a bound that stays valid when
            # this call is replayed from a graph at later context lengths
            o = tree_attention(q, self.k_pool, self.v_pool, self.block_tables, base_i, lvl_masks,
                               layer=li, max_keys=self.max_slots, workspace=self.attn_ws,
                               first_node=lo)
            delta = self._mm(o.view(B * n, Hq * hd), L["wo"])
            rmsnorm_(h, delta, L["ffn_norm"], s.eps, x)
            delta = self._mm(self._ffn_up(x, L["wgu"]), L["wdown"])
        rmsnorm_(h, delta, self.norm, s.eps, x)
        return (x @ self.lm_head).float().view(B, n, s.vocab)

    def commit(self, base: torch.Tensor, paths: torch.Tensor, path_lens: torch.Tensor) -> None:
        """Move the accepted nodes (slot base + node) to base + j in every
        layer (cfa_kv_commit, on the device)."""
        kv_commit(self.k_pool, self.v_pool, self.block_tables, base.to(torch.int32), paths,
                  path_lens)


# ---------------------------------------------------------------------------
# the step
# ---------------------------------------------------------------------------

@dataclass
class StepResult:
    path_len: List[int]          # 1 + accepted drafts, per sequence
    emitted: List[List[int]]     # accepted draft tokens then the final token
    final: List[int]


class TreeSpeculator:
    """Batched tree speculation: a binary draft tree of `depth` levels below
    the root (2^(depth+1) - 1 nodes), the last emitted token as its root."""

    def __init__(self, target: TargetModel, draft: DraftModel, B: int, context: int, *,
                 depth: int = 5, temperature: float = 1.0, mode: str = "cpp",
                 max_steps: int = 64, block_size: int = 16, seed: int = 0,
                 use_graphs: bool = False):
        dev = target.embed.device
        self.use_graphs = use_graphs
        self._graphs: dict = {}
        self.t, self.d = target, draft
        self.B, self.depth, self.T, self.mode = B, depth, temperature, mode
        self.N = 2 ** (depth + 1) - 1
        if self.N > 64:
            raise ValueError("a tree has at most 64 nodes")
        # uniforms per sequence and step: the walk draws one per tested child
        # (at most 2 per level) and one final draw, 2 * depth + 1 in all
        self.n_uniforms = 2 * 2 * depth + 2
        self.parents_np = T.binary_tree_parents(self.N)
        self.parents = torch.from_numpy(self.parents_np).to(dev)
        self.depths = torch.from_numpy(T.depths(self.parents_np)).to(dev)
        anc = T.ancestor_masks(self.parents_np)
        self.masks = T.mask_tensor(anc, dev)
        anc_bits = np.array([[(int(anc[i]) >> j) & 1 for j in range(self.N)]
                             for i in range(self.N)], bool)
        self.anc = torch.from_numpy(anc_bits).to(dev)           # [N, N]
        s = target.shape
        slots = context + self.N + 8 * max_steps
        nblk = B * (slots // block_size + 2) + 8
        cfg = KVCacheConfig(num_layers=s.n_layers, num_kv_heads=s.n_kv_heads,
                            head_dim=s.head_dim, block_size=block_size, total_gpu_blocks=nblk,
                            enable_prefix_caching=False, max_supported_batch_size=B,
                            max_blocks_per_sequence=slots // block_size + 2)
        self.kv = PagedKVCache(cfg, device=dev)
        self.gen = torch.Generator(device=dev).manual_seed(seed)
        # synthetic context: page tables for `context` tokens, N(0,1) K/V
        rng = np.random.default_rng(seed)
        for b in range(B):
            self.kv.register_sequence_with_prefix(b, rng.integers(0, s.vocab, context).tolist())
        self.kv.key_pool.normal_(generator=self.gen)
        self.kv.value_pool.normal_(generator=self.gen)
        draft.k_pool.normal_(generator=self.gen)
        draft.v_pool.normal_(generator=self.gen)
        self.ctx = [context] * B
        self.root = torch.randint(0, s.vocab, (B,), device=dev, generator=self.gen,
                                  dtype=torch.int32)
        self.draft_rows = torch.zeros(B, self.N, s.vocab, dtype=torch.float32, device=dev)
        self.max_slots = draft.max_slots

    def _level_forward(self, lvl: int, base: torch.Tensor, toks: torch.Tensor) -> torch.Tensor:
        """Draft logits [B, n, V] of the nodes of level `lvl` (tokens toks
        [B, n]), each seeing the context and its ancestors' tree slots."""
        lo, hi = 2 ** lvl - 1, 2 ** (lvl + 1) - 1
        pos = base[:, None] + self.depths[lo:hi][None, :]
        return self.d.forward_level(toks, pos, base, lo, self.masks)

    def _level_graph(self, lvl: int, base: torch.Tensor, toks: torch.Tensor) -> torch.Tensor:
        """_level_forward replayed from a HIP graph captured on first use
        (static base / token buffers; every other tensor it touches is
        persistent: weights, the draft KV cache, the graph's own pool)."""
        if lvl not in self._graphs:
            sb = base.clone()
            st = toks.clone()
            side = torch.cuda.Stream(base.device)
            side.wait_stream(torch.cuda.current_stream(base.device))
            with torch.cuda.stream(side):
                self._level_forward(lvl, sb, st)                # warm-up outside capture
            torch.cuda.current_stream(base.device).wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                out = self._level_forward(lvl, sb, st)
            self._graphs[lvl] = (g, sb, st, out)
        g, sb, st, out = self._graphs[lvl]
        sb.copy_(base)
        st.copy_(toks)
        g.replay()
        return out

    def propose(self, base: torch.Tensor) -> torch.Tensor:
        """Draft tree tokens [B, N] (node 0 = root); fills self.draft_rows
        with the draft logits of every expanded node."""
        B, dev = self.B, self.root.device
        tokens = torch.empty(B, self.N, dtype=torch.int32, device=dev)
        tokens[:, 0] = self.root
        for lvl in range(self.depth):
            lo, hi = 2 ** lvl - 1, 2 ** (lvl + 1) - 1
            run = self._level_graph if self.use_graphs else self._level_forward
            logits = run(lvl, base, tokens[:, lo:hi].contiguous())
            self.draft_rows[:, lo:hi] = logits
            kids = expand_tree_level(logits.view(B * (hi - lo), -1), children=2,
                                     mode="sample" if self.mode == "cpp" else "greedy",
                                     temperature=self.T, generator=self.gen)
            tokens[:, 2 * lo + 1: 2 * hi + 1] = kids.view(B, 2 * (hi - lo))
        return tokens

    def step(self, phase_ms: Optional[dict] = None) -> StepResult:
        """One verify step.  With `phase_ms`, the device time of each phase
        (propose, target, verify, commit) is added to it, in ms."""
        B, dev, N = self.B, self.root.device, self.N
        if max(self.ctx) + N > self.max_slots:
            raise RuntimeError("draft cache full: raise max_steps")
        ev = []

        def mark():
            if phase_ms is not None:
                e = torch.cuda.Event(enable_timing=True)
                e.record()
                ev.append(e)

        mark()
        base = torch.tensor(self.ctx, dtype=torch.int32, device=dev)
        tokens = self.propose(base)
        mark()
        for b in range(B):
            self.kv.append_tokens(b, N)
        desc = self.kv.prepare_batch_metadata(list(range(B)))
        pos = base[:, None] + self.depths[None, :]
        max_keys = max(self.ctx) + N
        logits = self.t.forward_tree(tokens, pos, self.kv, desc.block_tables, base, self.masks,
                                     max_keys)
        mark()
        u = 1.0 - torch.rand(B, self.n_uniforms, device=dev, generator=self.gen)
        res = tree_verify(logits, self.draft_rows, self.parents, tokens, u, input_kind="logits",
                          temperature=self.T, mode=self.mode)
        mark()
        try:
            check_status(res.status)
        except RuntimeError:
            # nothing is committed: the appended tree slots are released and
            # the context, root and both caches stay as they were
            for b in range(B):
                self.kv.truncate_sequence(b, self.ctx[b])
            raise
        new_lens = self.kv.commit_tree_paths(list(range(B)), desc, base, res.path, res.path_len)
        plen = [n - c for n, c in zip(new_lens, self.ctx)]
        self.d.commit(base, res.path, res.path_len)
        toks = res.tokens.cpu().tolist()
        ne = res.num_emitted.cpu().tolist()
        final = res.final.cpu().tolist()
        self.ctx = new_lens
        self.root = res.final.to(torch.int32)
        mark()
        if phase_ms is not None:
            torch.cuda.synchronize()
            for name, a, b in zip(("propose", "target", "verify", "commit"), ev[:-1], ev[1:]):
                phase_ms[name] = phase_ms.get(name, 0.0) + a.elapsed_time(b)
        return StepResult(path_len=plen, emitted=[t[:e] for t, e in zip(toks, ne)], final=final)
