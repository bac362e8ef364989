"""GPU tier: the model-scale verify step (cudaforge_amd/spec_step.py) at
small shapes.  The target's tree forward (W4A16 GEMMs, paged KV writes, tree
attention kernel) against an fp32 PyTorch forward over gathered pages with an
explicit tree mask; a few full steps checked for bookkeeping (context growth,
page tables, emitted tokens on the accepted path, draft-cache commit)."""
import math

import numpy as np
import pytest
import torch

from cudaforge_amd import tree as T
from cudaforge_amd.spec_step import (DraftModel, LlamaShape, TargetModel, TreeSpeculator,
                                     deinterleave_gate_up)
from cudaforge_amd.w4a16 import w4a16_dequant

pytestmark = pytest.mark.gpu

SMALL_T = LlamaShape(2, 256, 4, 2, 128, 384, 1000)
SMALL_D = LlamaShape(2, 128, 4, 2, 64, 256, 1000)


def _ref_forward(tm: TargetModel, tokens, positions, kv, tables, base, N):
    """fp32 reference of TargetModel.forward_tree given the pool contents
    before the call (the tree's own K/V come from this forward)."""
    s = tm.shape
    B = tokens.shape[0]
    hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
    G = Hq // Hkv
    par = T.binary_tree_parents(N)
    anc = T.ancestor_masks(par)
    allow = torch.tensor([[bool((int(anc[i]) >> j) & 1) for j in range(N)] for i in range(N)],
                         device=tokens.device)
    bs = kv.get_config().block_size

    def W(lin):
        return w4a16_dequant(lin.qweight, lin.scales, lin.zeros, group_size=lin.group,
                             dtype=torch.bfloat16).float()

    def rms(x, w):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + s.eps) * w.float()

    def rope(x, pos):
        D = x.shape[-1]
        inv = s.rope_theta ** (-torch.arange(0, D, 2, device=x.device, dtype=torch.float32) / D)
        ang = pos.float()[..., None] * inv
        cos = torch.cat([ang.cos(), ang.cos()], -1)[..., None, :]
        sin = torch.cat([ang.sin(), ang.sin()], -1)[..., None, :]
        rot = torch.cat([-x[..., D // 2:], x[..., : D // 2]], -1)
        return x * cos + rot * sin

    h = tm.embed[tokens.reshape(-1).long()].float()
    for li, L in enumerate(tm.layers):
        x = rms(h, L["attn_norm"])
        qkv = (x @ W(L["wqkv"])).view(B, N, Hq + 2 * Hkv, hd)
        q = rope(qkv[:, :, :Hq], positions)
        k = rope(qkv[:, :, Hq:Hq + Hkv], positions)
        v = qkv[:, :, Hq + Hkv:]
        o = torch.empty(B, N, Hq, hd, device=tokens.device)
        for b in range(B):
            ctx = int(base[b])
            pos = torch.arange(ctx, device=tokens.device)
            blk = tables[b].long()[pos // bs]
            kc = kv.key_pool[blk, li][torch.arange(ctx), :, pos % bs].float()
            vc = kv.value_pool[blk, li][torch.arange(ctx), :, pos % bs].float()
            kk = torch.cat([kc, k[b]], 0)
            vv = torch.cat([vc, v[b]], 0)
            mask = torch.ones(N, ctx + N, dtype=torch.bool, device=tokens.device)
            mask[:, ctx:] = allow
            for hh in range(Hq):
                sc = (q[b, :, hh] @ kk[:, hh // G].T) / math.sqrt(hd)
                sc = sc.masked_fill(~mask, float("-inf"))
                o[b, :, hh] = torch.softmax(sc, -1) @ vv[:, hh // G]
        h = h + o.reshape(B * N, Hq * hd) @ W(L["wo"])
        x = rms(h, L["ffn_norm"])
        gu = deinterleave_gate_up(x @ W(L["wgu"]))           # stored gate/up-interleaved
        h = h + (torch.nn.functional.silu(gu[:, : s.ffn]) * gu[:, s.ffn:]) @ W(L["wdown"])
    h = rms(h, tm.norm)
    return (h @ tm.lm_head.float()).view(B, N, s.vocab)


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def _rope(x, pos, theta):
    D = x.shape[-1]
    inv = theta ** (-torch.arange(0, D, 2, device=x.device, dtype=torch.float32) / D)
    ang = pos.float()[..., None] * inv
    cos = torch.cat([ang.cos(), ang.cos()], -1)[..., None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[..., None, :]
    rot = torch.cat([-x[..., D // 2:], x[..., : D // 2]], -1)
    return x * cos + rot * sin


def _ref_draft_level(dm: DraftModel, tokens, positions, base, lo, N):
    """fp32 reference of DraftModel.forward_level for tree nodes lo..lo+n-1 of
    an N-node binary tree, given the pool contents before the call (context
    and nodes < lo from the pools, this level's K/V from this forward)."""
    s = dm.shape
    B, n = tokens.shape
    hi = lo + n
    hd, Hq, Hkv = s.head_dim, s.n_heads, s.n_kv_heads
    G = Hq // Hkv
    anc = T.ancestor_masks(T.binary_tree_parents(N))
    allow = torch.tensor([[bool((int(anc[i]) >> j) & 1) for j in range(hi)] for i in range(lo, hi)],
                         device=tokens.device)
    bs = dm.block_size
    h = dm.embed[tokens.reshape(-1).long()].float()
    for li, L in enumerate(dm.layers):
        x = _rms(h, L["attn_norm"], s.eps)
        qkv = (x @ L["wqkv"].float()).view(B, n, Hq + 2 * Hkv, hd)
        q = _rope(qkv[:, :, :Hq], positions, s.rope_theta)
        k = _rope(qkv[:, :, Hq:Hq + Hkv], positions, s.rope_theta)
        v = qkv[:, :, Hq + Hkv:]
        o = torch.empty(B, n, Hq, hd, device=tokens.device)
        for b in range(B):
            ctx = int(base[b])
            old = torch.arange(ctx + lo, device=tokens.device)
            blk = dm.block_tables[b].long()[old // bs]
            kc = dm.k_pool[blk, li][torch.arange(ctx + lo), :, old % bs].float()
            vc = dm.v_pool[blk, li][torch.arange(ctx + lo), :, old % bs].float()
            kk = torch.cat([kc, k[b]], 0)
            vv = torch.cat([vc, v[b]], 0)
            mask = torch.ones(n, ctx + hi, dtype=torch.bool, device=tokens.device)
            mask[:, ctx:] = allow
            for hh in range(Hq):
                sc = (q[b, :, hh] @ kk[:, hh // G].T) / math.sqrt(hd)
                sc = sc.masked_fill(~mask, float("-inf"))
                o[b, :, hh] = torch.softmax(sc, -1) @ vv[:, hh // G]
        h = h + o.reshape(B * n, Hq * hd) @ L["wo"].float()
        x = _rms(h, L["ffn_norm"], s.eps)
        gu = deinterleave_gate_up(x @ L["wgu"].float())     # stored gate/up-interleaved
        h = h + (torch.nn.functional.silu(gu[:, : s.ffn]) * gu[:, s.ffn:]) @ L["wdown"].float()
    h = _rms(h, dm.norm, s.eps)
    return (h @ dm.lm_head.float()).view(B, n, s.vocab)


def test_draft_levels_vs_fp32(device):
    """The drafter's level forwards (paged pools, tree-attention kernel at
    head_dim 64 on the level's nodes) against an fp32 forward over gathered
    pages, level by level as propose() runs them."""
    B, ctx0, depth = 3, 40, 3
    N = 2 ** (depth + 1) - 1
    tm = TargetModel(SMALL_T, device, seed=9)
    dm = DraftModel(SMALL_D, device, B, max_slots=ctx0 + 64 + 64)
    sp = TreeSpeculator(tm, dm, B, ctx0, depth=depth, max_steps=8, seed=10)
    base = torch.tensor([40, 23, 57], dtype=torch.int32, device=device)
    for lvl in range(depth):
        lo, hi = 2 ** lvl - 1, 2 ** (lvl + 1) - 1
        toks = torch.randint(0, SMALL_D.vocab, (B, hi - lo), device=device, dtype=torch.int32)
        pos = base[:, None] + sp.depths[lo:hi][None, :]
        want = _ref_draft_level(dm, toks, pos, base, lo, N)
        got = sp._level_forward(lvl, base, toks)
        torch.cuda.synchronize()
        err = (got - want).abs().max().item()
        scale = want.abs().max().item()
        assert err <= 3e-2 * max(1.0, scale), (lvl, err, scale)


def test_target_tree_forward_vs_fp32(device):
    B, ctx0, N = 3, 50, 15
    tm = TargetModel(SMALL_T, device, seed=3)
    dm = DraftModel(SMALL_D, device, B, max_slots=ctx0 + 64 + 64)
    sp = TreeSpeculator(tm, dm, B, ctx0, depth=3, temperature=1.0, max_steps=8, seed=4)
    sp.ctx = [50, 37, 45]
    for b in range(B):
        sp.kv.truncate_sequence(b, sp.ctx[b])
    base = torch.tensor(sp.ctx, dtype=torch.int32, device=device)
    tokens = torch.randint(0, SMALL_T.vocab, (B, N), device=device, dtype=torch.int32,
                           generator=torch.Generator(device=device).manual_seed(21))
    for b in range(B):
        sp.kv.append_tokens(b, N)
    desc = sp.kv.prepare_batch_metadata(list(range(B)))
    pos = base[:, None] + sp.depths[None, :]
    want = _ref_forward(tm, tokens, pos, sp.kv, desc.block_tables, base, N)
    got = tm.forward_tree(tokens, pos, sp.kv, desc.block_tables, base, sp.masks, max(sp.ctx) + N)
    torch.cuda.synchronize()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    assert err <= 3e-2 * max(1.0, scale), (err, scale)


def test_target_tree_forward_8b_width_vs_fp32(device):
    """The target's tree forward at the 8B layer width (d 4096, GQA 32/8,
    head_dim 128, FFN 14336, V 128256) with 2 of its 32 layers, over the full
    63-node tree, against the fp32 forward."""
    shape = LlamaShape(2, 4096, 32, 8, 128, 14336, 128256)
    B, ctx0, N = 2, 130, 63
    tm = TargetModel(shape, device, seed=13)
    dm = DraftModel(LlamaShape(1, 128, 4, 2, 64, 256, 128256), device, B,
                    max_slots=ctx0 + 64 + 64)
    sp = TreeSpeculator(tm, dm, B, ctx0, depth=5, temperature=1.0, max_steps=8, seed=14)
    sp.ctx = [130, 77]
    for b in range(B):
        sp.kv.truncate_sequence(b, sp.ctx[b])
    base = torch.tensor(sp.ctx, dtype=torch.int32, device=device)
    tokens = torch.randint(0, shape.vocab, (B, N), device=device, dtype=torch.int32,
                           generator=torch.Generator(device=device).manual_seed(22))
    for b in range(B):
        sp.kv.append_tokens(b, N)
    desc = sp.kv.prepare_batch_metadata(list(range(B)))
    pos = base[:, None] + sp.depths[None, :]
    got = tm.forward_tree(tokens, pos, sp.kv, desc.block_tables, base, sp.masks, max(sp.ctx) + N)
    torch.cuda.synchronize()
    got = got.float()
    want = _ref_forward(tm, tokens, pos, sp.kv, desc.block_tables, base, N)
    torch.cuda.synchronize()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    assert err <= 3e-2 * max(1.0, scale), (err, scale)


def _slots(pool, table, n):
    """Slots [0, n) of one sequence of a paged pool [blocks, L, Hkv, bs, D]
    as [L, Hkv, n, D]."""
    pages = pool[table.long()]
    P, L, H, bs, D = pages.shape
    return pages.permute(1, 2, 0, 3, 4).reshape(L, H, P * bs, D)[:, :, :n]


def test_full_8b_step_bookkeeping(device):
    """Two verify steps of the full workload (32-layer 8B-shape W4A16 target,
    1B-shape draft, B = 8, context 2048, 63-node tree): paths, context growth,
    page tables, emitted ids and the draft cache's commit."""
    from cudaforge_amd.spec_step import DRAFT_1B, TARGET_8B

    B, ctx0 = 8, 2048
    tm = TargetModel(TARGET_8B, device, seed=0)
    dm = DraftModel(DRAFT_1B, device, B, max_slots=ctx0 + 64 + 8 * 4)
    sp = TreeSpeculator(tm, dm, B, ctx0, depth=5, temperature=1.0, mode="cpp", max_steps=4,
                        use_graphs=True)
    for _ in range(2):
        ctx_before = list(sp.ctx)
        dk_before = dm.k_pool.clone()
        r = sp.step()
        torch.cuda.synchronize()
        for b in range(B):
            L = r.path_len[b]
            assert 1 <= L <= sp.depth + 1
            assert sp.ctx[b] == ctx_before[b] + L
            assert sp.kv.context_length(b) == sp.ctx[b]
            assert len(sp.kv.get_block_table(b)) == -(-sp.ctx[b] // 16)
            assert len(r.emitted[b]) == L and r.emitted[b][-1] == r.final[b]
            assert all(0 <= t < TARGET_8B.vocab for t in r.emitted[b])
            # the draft cache below the old context is untouched by the step
            assert torch.equal(_slots(dk_before, dm.block_tables[b], ctx_before[b]),
                               _slots(dm.k_pool, dm.block_tables[b], ctx_before[b]))
        assert sp.root.tolist() == r.final
    del sp, tm, dm
    torch.cuda.empty_cache()


@pytest.mark.parametrize("mode", ["cpp", "greedy"])
def test_steps_bookkeeping(device, mode):
    B, ctx0 = 4, 40
    tm = TargetModel(SMALL_T, device, seed=5)
    dm = DraftModel(SMALL_D, device, B, max_slots=ctx0 + 64 + 8 * 8)
    sp = TreeSpeculator(tm, dm, B, ctx0, depth=3, temperature=0.8, mode=mode, max_steps=8, seed=6)
    for _ in range(3):
        ctx_before = list(sp.ctx)
        base = torch.tensor(ctx_before, dtype=torch.int32, device=device)
        r = sp.step()
        torch.cuda.synchronize()
        for b in range(B):
            L = r.path_len[b]
            assert 1 <= L <= sp.depth + 1
            assert sp.ctx[b] == ctx_before[b] + L
            assert sp.kv.context_length(b) == sp.ctx[b]
            assert len(sp.kv.get_block_table(b)) == -(-sp.ctx[b] // 16)
            assert len(r.emitted[b]) == L and r.emitted[b][-1] == r.final[b]
        assert sp.root.tolist() == r.final


def test_draft_level_graphs_match_eager(device):
    """The draft levels replayed from HIP graphs give the eager logits, on
    every replay (several steps, eager work in between)."""
    B, ctx0 = 3, 30
    tm = TargetModel(SMALL_T, device, seed=7)
    dm = DraftModel(SMALL_D, device, B, max_slots=ctx0 + 64 + 8 * 8)
    sp = TreeSpeculator(tm, dm, B, ctx0, depth=3, max_steps=8, seed=8, use_graphs=True)
    for rep in range(4):
        base = torch.tensor([ctx0 + 2 * rep, ctx0 + rep, ctx0], dtype=torch.int32, device=device)
        for lvl in range(3):
            n = 2 ** lvl
            toks = torch.randint(0, SMALL_D.vocab, (B, n), device=device, dtype=torch.int32)
            k0, v0 = dm.k_pool.clone(), dm.v_pool.clone()
            eager = sp._level_forward(lvl, base, toks).clone()
            k1, v1 = dm.k_pool.clone(), dm.v_pool.clone()
            dm.k_pool.copy_(k0)
            dm.v_pool.copy_(v0)
            graph = sp._level_graph(lvl, base, toks).clone()
            torch.cuda.synchronize()
            assert torch.equal(graph, eager), (rep, lvl, (graph - eager).abs().max().item())
            assert torch.equal(dm.k_pool, k1) and torch.equal(dm.v_pool, v1)


@pytest.mark.parametrize("status", [1, 2])
def test_failed_tree_verification_raises_and_commits_nothing(device, monkeypatch, status):
    """A tree verification that reports a failure (1: the uniform stream ran
    out, driven for real by a one-uniform stream; 2: a team wait timed out,
    forced on the host by setting the status the kernel returned) raises
    RuntimeError before anything is committed: context, root, page tables,
    committed K/V of both caches unchanged; the next step runs normally.  The
    reference raises rather than return unusable results
    (speculative.cpp:58-62)."""
    import cudaforge_amd.spec_step as S

    B, ctx0 = 3, 40
    tm = TargetModel(SMALL_T, device, seed=15)
    dm = DraftModel(SMALL_D, device, B, max_slots=ctx0 + 64 + 8 * 8)
    sp = TreeSpeculator(tm, dm, B, ctx0, depth=3, temperature=0.8, mode="cpp", max_steps=8,
                        seed=16)
    sp.step()
    torch.cuda.synchronize()
    ctx, root = list(sp.ctx), sp.root.clone()
    tables = [list(sp.kv.get_block_table(b)) for b in range(B)]
    kt = [_slots(sp.kv.key_pool, torch.tensor(tables[b], device=device), ctx[b]).clone()
          for b in range(B)]
    dk = [_slots(dm.k_pool, dm.block_tables[b], ctx[b]).clone() for b in range(B)]
    if status == 1:
        sp.n_uniforms = 1
    else:
        real = S.tree_verify

        def timed_out(*a, **k):
            out = real(*a, **k)
            out.status[1] = 2
            return out

        monkeypatch.setattr(S, "tree_verify", timed_out)
    with pytest.raises(RuntimeError, match="ran out" if status == 1 else "timed out"):
        sp.step()
    torch.cuda.synchronize()
    assert sp.ctx == ctx and torch.equal(sp.root, root)
    for b in range(B):
        assert sp.kv.context_length(b) == ctx[b]
        assert list(sp.kv.get_block_table(b)) == tables[b]
        assert torch.equal(_slots(sp.kv.key_pool, torch.tensor(tables[b], device=device),
                                  ctx[b]), kt[b])
        assert torch.equal(_slots(dm.k_pool, dm.block_tables[b], ctx[b]), dk[b])
    sp.n_uniforms = 2 * 2 * sp.depth + 2
    monkeypatch.undo()
    r = sp.step()
    for b in range(B):
        assert sp.ctx[b] == ctx[b] + r.path_len[b] and sp.kv.context_length(b) == sp.ctx[b]
