"""Tensor-level entry points of the verification path (PyTorch-ROCm host side).

Each function validates shapes, dtypes, devices and strides on the host,
allocates outputs and workspace with torch's caching allocator, and calls one
C-ABI entry point of ``libcfa.so`` on torch's current HIP stream.  Nothing here
computes on the CPU: without the HIP library every call raises.

Reference semantics (paths inside Bahaa-Labs/CUDAForge):
  chain_verify, mode="cpp"     csrc/src/scheduler/speculative.cpp:50-103
  chain_verify, mode="greedy"  csrc/src/scheduler/speculative.cpp:105-150
  chain_verify, mode="python"  cudaforge/speculative.py:152-195
  tree_attention               paged layout of csrc/src/memory/paged_kv_cache.cpp:
                               13-21, 409-421; descriptor of paged_kv_cache.h:81-94
  kv_commit                    device half of append_tokens, paged_kv_cache.cpp:255-286
  tree_verify                  speculative.cpp:50-150 generalised to a draft tree
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

_MODES = {"cpp": _lib.CFA_MODE_CPP, "python": _lib.CFA_MODE_PYTHON, "greedy": _lib.CFA_MODE_GREEDY}
_KINDS = {"probs": _lib.CFA_INPUT_PROBS, "logits": _lib.CFA_INPUT_LOGITS}


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_cuda(name: str, t: torch.Tensor, dtype: torch.dtype, device=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a HIP device tensor (got {t.device})")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")


@dataclass
class ChainVerifyOutput:
    """Per-sequence results of one chain verification (all int32 device tensors).

    accept_len   [B]      accepted draft tokens (python mode: the batch-wide n)
    tokens       [B, K+1] accepted drafts then the final token, -1 padded
    num_emitted  [B]      valid entries of ``tokens``
    final        [B]      the resampled or bonus token (final_token)
    eos          [B]      end_of_sequence flag (cpp / greedy modes)
    target_probs / draft_probs  the fp32 probabilities the decisions used, when
                          ``return_probs`` was set
    """

    accept_len: torch.Tensor
    tokens: torch.Tensor
    num_emitted: torch.Tensor
    final: torch.Tensor
    eos: torch.Tensor
    target_probs: Optional[torch.Tensor] = None
    draft_probs: Optional[torch.Tensor] = None


def chain_workspace_bytes(B: int, K: int, V: int, input_kind: str = "logits",
                          mode: str = "cpp") -> int:
    return int(_lib.load().cfa_chain_verify_workspace_size(B, K, V, _KINDS[input_kind],
                                                            _MODES[mode]))


def chain_verify(target: torch.Tensor, draft: Optional[torch.Tensor],
                 draft_tokens: torch.Tensor, uniforms: Optional[torch.Tensor], *,
                 input_kind: str = "logits", temperature: float = 1.0, top_p: float = 1.0,
                 mode: str = "cpp", eos_token_id: int = -1, return_probs: bool = False,
                 workspace: Optional[torch.Tensor] = None) -> ChainVerifyOutput:
    """Verify B chains of K draft tokens in one pass over the logits.

    target [B, K+1, V] fp32 and draft [B, K, V] fp32 (None in greedy mode) may be
    strided views (the last dimension must be contiguous); draft_tokens [B, K]
    int32; uniforms fp32 in [0, 1): [B, K+1] in cpp mode, [B, K+2] in python
    mode (column K+1 drives the bonus that follows a rejection at the last
    position, speculative.py:188), None in greedy mode.

    input_kind "logits": probabilities are softmax(row / temperature), fused
    into the kernel; "probs": rows are probabilities (temperature unused).
    """
    if mode not in _MODES:
        raise ValueError(f"mode must be one of {sorted(_MODES)}")
    if input_kind not in _KINDS:
        raise ValueError(f"input_kind must be one of {sorted(_KINDS)}")
    _require_cuda("target", target, torch.float32)
    dev = target.device
    if target.dim() != 3:
        raise ValueError("target must be [B, K+1, V]")
    B, K1, V = target.shape
    K = K1 - 1
    if B <= 0 or V <= 0 or K < 0:
        raise ValueError("target must be [B, K+1, V] with B, V > 0")
    if target.stride(2) != 1:
        raise ValueError("target's vocabulary dimension must be contiguous")
    _require_cuda("draft_tokens", draft_tokens, torch.int32, dev)
    if tuple(draft_tokens.shape) != (B, K):
        raise ValueError(f"draft_tokens must be [B, K] = [{B}, {K}]")
    draft_tokens = draft_tokens.contiguous()
    greedy = mode == "greedy"
    if not greedy:
        if draft is None or uniforms is None:
            raise ValueError("draft and uniforms are required outside greedy mode")
        _require_cuda("draft", draft, torch.float32, dev)
        if tuple(draft.shape) != (B, K, V):
            raise ValueError("Incompatible draft and target tensor dimensions in SpeculativeEngine.")
        if K > 0 and draft.stride(2) != 1:
            raise ValueError("draft's vocabulary dimension must be contiguous")
        _require_cuda("uniforms", uniforms, torch.float32, dev)
        nu = K + 2 if mode == "python" else K + 1
        if tuple(uniforms.shape) != (B, nu):
            cols = "K+2" if mode == "python" else "K+1"
            raise ValueError(f"uniforms must be [B, {cols}] = [{B}, {nu}] in {mode} mode")
        uniforms = uniforms.contiguous()
    if input_kind == "logits" and not temperature > 0.0:
        raise ValueError("temperature must be > 0")

    lib = _lib.load()
    ws_need = int(lib.cfa_chain_verify_workspace_size(B, K, V, _KINDS[input_kind], _MODES[mode]))
    if workspace is None or workspace.numel() < ws_need:
        workspace = torch.empty(max(ws_need, 1), dtype=torch.uint8, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    out = ChainVerifyOutput(
        accept_len=torch.empty(B, **i32), tokens=torch.empty(B, K + 1, **i32),
        num_emitted=torch.empty(B, **i32), final=torch.empty(B, **i32),
        eos=torch.empty(B, **i32))
    if return_probs:
        out.target_probs = torch.empty(B, K + 1, V, dtype=torch.float32, device=dev)
        if not greedy and K > 0:
            out.draft_probs = torch.empty(B, K, V, dtype=torch.float32, device=dev)
    d_sb = d_sk = 0
    if draft is not None and not greedy:
        d_sb, d_sk = draft.stride(0), draft.stride(1)
        if K == 0:
            d_sb = d_sk = V
    with torch.cuda.device(dev):
        rc = lib.cfa_chain_verify(
            target.data_ptr(), target.stride(0), target.stride(1),
            None if greedy or draft is None else draft.data_ptr(), d_sb, d_sk,
            _KINDS[input_kind], draft_tokens.data_ptr(),
            None if uniforms is None else uniforms.data_ptr(),
            B, K, V, ctypes.c_float(temperature), ctypes.c_float(top_p), _MODES[mode],
            int(eos_token_id), out.accept_len.data_ptr(), out.tokens.data_ptr(),
            out.num_emitted.data_ptr(), out.final.data_ptr(), out.eos.data_ptr(),
            _ptr(out.target_probs), _ptr(out.draft_probs), workspace.data_ptr(),
            workspace.numel(), _stream_ptr(dev))
    _lib.check(rc, "cfa_chain_verify")
    return out


def tree_attention_workspace_bytes(B: int, N: int, n_q_heads: int, n_kv_heads: int,
                                   head_dim: int, max_keys: int, num_splits: int = 0) -> int:
    return int(_lib.load().cfa_tree_attention_workspace_size(B, N, n_q_heads, n_kv_heads,
                                                              head_dim, max_keys, num_splits))


def tree_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                   block_tables: torch.Tensor, ctx_lens: torch.Tensor,
                   tree_mask: torch.Tensor, *, layer: int = 0,
                   sm_scale: Optional[float] = None, max_keys: Optional[int] = None,
                   num_splits: int = 0, out: Optional[torch.Tensor] = None,
                   workspace: Optional[torch.Tensor] = None, first_node: int = 0) -> torch.Tensor:
    """Tree-masked attention of draft-tree nodes over a paged KV cache.

    q [B, Nq, Hq, D] bf16 (D = 128 or 64): the queries of tree nodes
    first_node .. first_node + Nq - 1 of an N = first_node + Nq node tree;
    k_pool / v_pool [num_blocks, num_layers, Hkv, block_size, D] bf16 (the
    reference's per-block layout); block_tables [B, max_blocks] int32;
    ctx_lens [B] int32 (tokens before the tree; the tree's K/V sit at
    ctx_len + i, i < N); tree_mask int64 [N] or [B, N] holding each node's
    64-bit ancestor-or-self mask.  max_keys bounds ctx_len + N on the host
    (computed with one sync when omitted).  Returns [B, Nq, Hq, D] bf16.
    """
    _require_cuda("q", q, torch.bfloat16)
    dev = q.device
    if q.dim() != 4:
        raise ValueError("q must be [B, Nq, Hq, D]")
    B, Nq, Hq, D = q.shape
    if first_node < 0:
        raise ValueError("first_node must be >= 0")
    N = first_node + Nq
    q = q.contiguous()
    for name, pool in (("k_pool", k_pool), ("v_pool", v_pool)):
        _require_cuda(name, pool, torch.bfloat16, dev)
        if pool.dim() != 5 or not pool.is_contiguous():
            raise ValueError(f"{name} must be a contiguous [blocks, layers, Hkv, block_size, D] tensor")
    if k_pool.shape != v_pool.shape:
        raise ValueError("k_pool and v_pool must have the same shape")
    nblk, nlayers, Hkv, bs, Dp = k_pool.shape
    if Dp != D:
        raise ValueError("head_dim of q and of the pools differ")
    _require_cuda("block_tables", block_tables, torch.int32, dev)
    if block_tables.dim() != 2 or block_tables.shape[0] != B:
        raise ValueError("block_tables must be [B, max_blocks]")
    block_tables = block_tables.contiguous()
    _require_cuda("ctx_lens", ctx_lens, torch.int32, dev)
    if tuple(ctx_lens.shape) != (B,):
        raise ValueError("ctx_lens must be [B]")
    ctx_lens = ctx_lens.contiguous()
    _require_cuda("tree_mask", tree_mask, torch.int64, dev)
    if tree_mask.dim() == 1 and tree_mask.shape[0] == N:
        mstride = 0
    elif tree_mask.dim() == 2 and tuple(tree_mask.shape) == (B, N):
        mstride = N
    else:
        raise ValueError("tree_mask must be [N] or [B, N]")
    tree_mask = tree_mask.contiguous()
    if sm_scale is None:
        sm_scale = D ** -0.5
    if max_keys is None:
        max_keys = int(ctx_lens.max().item()) + N
    if out is None:
        out = torch.empty_like(q)
    lib = _lib.load()
    need = int(lib.cfa_tree_attention_workspace_size(B, Nq, Hq, Hkv, D, max_keys, num_splits))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.cfa_tree_attention(
            q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), block_tables.data_ptr(),
            block_tables.shape[1], ctx_lens.data_ptr(), nblk, nlayers, int(layer), bs,
            tree_mask.data_ptr(), mstride, B, N, int(first_node), Hq, Hkv, D, ctypes.c_float(sm_scale),
            int(max_keys), int(num_splits), out.data_ptr(), workspace.data_ptr(),
            workspace.numel(), _stream_ptr(dev))
    _lib.check(rc, "cfa_tree_attention")
    return out


@dataclass
class KVCommitOutput:
    new_ctx_lens: torch.Tensor  # [B] int32: ctx_lens + path_len (unchanged when rejected)
    status: torch.Tensor        # [B] int32: 0 committed, 1 rejected (bad path or page)


def kv_commit(k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
              ctx_lens: torch.Tensor, paths: torch.Tensor, path_lens: torch.Tensor
              ) -> KVCommitOutput:
    """Move each sequence's accepted tree nodes (paths [B, P] int32, node ids
    with the root 0 first, path_lens [B]) from slots ctx + node to ctx + j in
    every layer and KV head of both pools (in place)."""
    for name, pool in (("k_pool", k_pool), ("v_pool", v_pool)):
        if not isinstance(pool, torch.Tensor) or pool.device.type != "cuda":
            raise ValueError(f"{name} must be a HIP device tensor")
        if pool.dim() != 5 or not pool.is_contiguous():
            raise ValueError(f"{name} must be a contiguous [blocks, layers, Hkv, block_size, D] tensor")
    if k_pool.shape != v_pool.shape or k_pool.dtype != v_pool.dtype:
        raise ValueError("k_pool and v_pool must match in shape and dtype")
    dev = k_pool.device
    nblk, nlayers, Hkv, bs, D = k_pool.shape
    _require_cuda("block_tables", block_tables, torch.int32, dev)
    B = block_tables.shape[0]
    for name, t, shape in (("ctx_lens", ctx_lens, (B,)), ("path_lens", path_lens, (B,))):
        _require_cuda(name, t, torch.int32, dev)
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must be [B]")
    _require_cuda("paths", paths, torch.int32, dev)
    if paths.dim() != 2 or paths.shape[0] != B:
        raise ValueError("paths must be [B, max_path]")
    block_tables, ctx_lens, paths, path_lens = (t.contiguous() for t in
                                                (block_tables, ctx_lens, paths, path_lens))
    out = KVCommitOutput(new_ctx_lens=torch.empty(B, dtype=torch.int32, device=dev),
                         status=torch.empty(B, dtype=torch.int32, device=dev))
    with torch.cuda.device(dev):
        rc = _lib.load().cfa_kv_commit(
            k_pool.data_ptr(), v_pool.data_ptr(), block_tables.data_ptr(), block_tables.shape[1],
            ctx_lens.data_ptr(), paths.data_ptr(), paths.shape[1], path_lens.data_ptr(), B, nblk,
            nlayers, Hkv, bs, D, k_pool.element_size(), out.new_ctx_lens.data_ptr(),
            out.status.data_ptr(), _stream_ptr(dev))
    _lib.check(rc, "cfa_kv_commit")
    return out


@dataclass
class TreeVerifyOutput:
    """Per-sequence results of tree verification (int32 device tensors)."""

    path: torch.Tensor         # [B, N] accepted node ids from the root, -1 padded
    path_len: torch.Tensor     # [B] 1 + accepted drafts
    tokens: torch.Tensor       # [B, N+1] accepted draft tokens then the final token
    num_emitted: torch.Tensor  # [B]
    final: torch.Tensor        # [B]
    eos: torch.Tensor          # [B]
    status: torch.Tensor       # [B] 0 ok, 1 uniforms ran out, 2 a team wait timed out
    target_probs: Optional[torch.Tensor] = None
    draft_probs: Optional[torch.Tensor] = None

    def check_status(self) -> None:
        """Raise RuntimeError unless every sequence's status is 0 (one host sync)."""
        check_status(self.status)


TREE_STATUS = {1: "the uniform stream ran out",
               2: "a wait between the work-groups of its team timed out (kernels of other "
                  "streams held a member back); run the call again"}


def check_status(status: torch.Tensor) -> None:
    """Raise RuntimeError when a tree verification reported a failure.

    status [B] int32 (``TreeVerifyOutput.status``): 0 ok, 1 the uniform
    stream ran out, 2 a team wait timed out.  The paths and tokens of a
    failed call are not valid and must not be committed; the reference raises
    rather than return unusable results (speculative.cpp:58-62).  Reads the
    status to the host: one synchronisation with its stream."""
    st = status.detach().to("cpu", torch.int32).reshape(-1)
    bad = torch.nonzero(st).reshape(-1).tolist()
    if not bad:
        return
    codes = sorted({int(st[b]) for b in bad})
    what = "; ".join(f"{TREE_STATUS.get(c, f'status {c}')} (sequences "
                     f"{[b for b in bad if int(st[b]) == c][:8]})" for c in codes)
    raise RuntimeError(f"cfa_tree_verify failed: {what}")


def tree_verify(target: torch.Tensor, draft: Optional[torch.Tensor], parents: torch.Tensor,
                node_tokens: torch.Tensor, uniforms: Optional[torch.Tensor], *,
                input_kind: str = "logits", temperature: float = 1.0, mode: str = "cpp",
                eos_token_id: int = -1, return_probs: bool = False,
                workspace: Optional[torch.Tensor] = None) -> TreeVerifyOutput:
    """Accept the longest root-to-leaf path of a draft tree.

    target / draft [B, N, V] fp32 (rows may be strided; the vocabulary
    dimension contiguous); parents [N] or [B, N] int32 with parents[c] < c and
    parents[0] = -1; node_tokens [B, N] int32; uniforms [B, n_u] fp32 (cpp mode).
    workspace: optional uint8 device tensor of tree_verify_workspace_bytes(B).
    status: 0 ok, 1 the uniform stream ran out, 2 a wait between the
    work-groups of a sequence timed out -- kernels of other streams held one
    of them back; run the call again.  ``check_status`` (or the output's
    ``check_status()``) raises RuntimeError on either; the call itself does
    not synchronise.
    """
    if mode not in ("cpp", "greedy"):
        raise ValueError("mode must be 'cpp' or 'greedy'")
    if input_kind not in _KINDS:
        raise ValueError(f"input_kind must be one of {sorted(_KINDS)}")
    _require_cuda("target", target, torch.float32)
    dev = target.device
    if target.dim() != 3 or target.stride(2) != 1:
        raise ValueError("target must be [B, N, V] with a contiguous last dimension")
    B, N, V = target.shape
    greedy = mode == "greedy"
    if not greedy:
        if draft is None or uniforms is None:
            raise ValueError("draft and uniforms are required in cpp mode")
        _require_cuda("draft", draft, torch.float32, dev)
        if tuple(draft.shape) != (B, N, V) or draft.stride(2) != 1:
            raise ValueError("draft must be [B, N, V] with a contiguous last dimension")
        _require_cuda("uniforms", uniforms, torch.float32, dev)
        if uniforms.dim() != 2 or uniforms.shape[0] != B:
            raise ValueError("uniforms must be [B, n_uniforms]")
        uniforms = uniforms.contiguous()
    _require_cuda("parents", parents, torch.int32, dev)
    if parents.dim() == 1 and parents.shape[0] == N:
        pstride = 0
    elif parents.dim() == 2 and tuple(parents.shape) == (B, N):
        pstride = N
    else:
        raise ValueError("parents must be [N] or [B, N]")
    parents = parents.contiguous()
    _require_cuda("node_tokens", node_tokens, torch.int32, dev)
    if tuple(node_tokens.shape) != (B, N):
        raise ValueError("node_tokens must be [B, N]")
    node_tokens = node_tokens.contiguous()
    if input_kind == "logits" and not temperature > 0.0:
        raise ValueError("temperature must be > 0")
    i32 = dict(dtype=torch.int32, device=dev)
    out = TreeVerifyOutput(path=torch.empty(B, N, **i32), path_len=torch.empty(B, **i32),
                           tokens=torch.empty(B, N + 1, **i32), num_emitted=torch.empty(B, **i32),
                           final=torch.empty(B, **i32), eos=torch.empty(B, **i32),
                           status=torch.empty(B, **i32))
    if return_probs:
        out.target_probs = torch.zeros(B, N, V, dtype=torch.float32, device=dev)
        if not greedy:
            out.draft_probs = torch.zeros(B, N, V, dtype=torch.float32, device=dev)
    lib = _lib.load()
    need = int(lib.cfa_tree_verify_workspace_size(B))
    if workspace is None or workspace.numel() < need or workspace.data_ptr() % 256:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.cfa_tree_verify(
            target.data_ptr(), target.stride(0), target.stride(1),
            None if greedy else draft.data_ptr(), 0 if greedy else draft.stride(0),
            0 if greedy else draft.stride(1), _KINDS[input_kind], parents.data_ptr(), pstride,
            node_tokens.data_ptr(), None if greedy else uniforms.data_ptr(),
            0 if greedy else uniforms.shape[1], B, N, V, ctypes.c_float(temperature),
            _MODES[mode], int(eos_token_id), out.path.data_ptr(), out.path_len.data_ptr(),
            out.tokens.data_ptr(), out.num_emitted.data_ptr(), out.final.data_ptr(),
            out.eos.data_ptr(), out.status.data_ptr(), _ptr(out.target_probs),
            _ptr(out.draft_probs), workspace.data_ptr(), workspace.numel(), _stream_ptr(dev))
    _lib.check(rc, "cfa_tree_verify")
    return out


def tree_verify_workspace_bytes(B: int) -> int:
    return int(_lib.load().cfa_tree_verify_workspace_size(B))
