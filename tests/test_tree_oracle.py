"""CPU tier: pin the tree oracles (oracle/oracle.py tree_attention,
gather_pages, kv_commit, context_length) and the host tree helpers against
closed forms and library routines (torch SDPA, index_copy)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from cudaforge_amd import tree as T
from oracle import oracle as O
from tests import helpers as H


def test_binary_tree_masks_known_answers():
    p = T.binary_tree_parents(7)
    assert list(p) == [-1, 0, 0, 1, 1, 2, 2]
    m = T.ancestor_masks(p)
    assert [int(x) for x in m] == [0b1, 0b11, 0b101, 0b1011, 0b10011, 0b100101, 0b1000101]
    assert list(T.depths(p)) == [0, 1, 1, 2, 2, 2, 2]
    p63 = T.binary_tree_parents(63)
    d = T.depths(p63)
    assert list(d) == [int(np.floor(np.log2(i + 1))) for i in range(63)]
    assert all(bin(int(x)).count("1") == dd + 1 for x, dd in zip(T.ancestor_masks(p63), d))
    # the oracle's restatement agrees with the package helper
    assert np.array_equal(O.ancestor_masks(p63), T.ancestor_masks(p63))


def test_tree_validation():
    with pytest.raises(ValueError):
        T.ancestor_masks([0, 0])
    with pytest.raises(ValueError):
        T.ancestor_masks([-1, 1])
    with pytest.raises(ValueError):
        T.ancestor_masks([-1] + [0] * 64)


def test_context_length_reference_kat():
    # tests/cpp/test_paged_kv_cache.cpp:39-74: prompts of 32 and 48 tokens in
    # 16-token blocks give context lengths 32 and 48
    assert O.context_length(2, 16, 16) == 32
    assert O.context_length(3, 16, 16) == 48
    assert O.context_length(1, 16, 5) == 5


def test_gather_pages_inverts_scatter():
    g = torch.Generator().manual_seed(1)
    K = [torch.randn(L, 2, 8, generator=g) for L in (37, 16, 5)]
    kp, vp, bt = H.paged_pools(K, K, block_size=16, num_layers=2, layer=1)
    for b, k in enumerate(K):
        got = O.gather_pages(kp, bt[b], k.shape[0], 1, 16)
        assert torch.equal(got, k)


def _ref_sdpa(q, k, v, mask, scale):
    # q [N, H, D], k/v [L, Hkv, D] -> SDPA per head with GQA broadcast, fp64
    N, Hq, D = q.shape
    g = Hq // k.shape[1]
    kk = k.repeat_interleave(g, dim=1).permute(1, 0, 2).double()
    vv = v.repeat_interleave(g, dim=1).permute(1, 0, 2).double()
    qq = q.permute(1, 0, 2).double()
    o = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=scale)
    return o.permute(1, 0, 2)


@pytest.mark.parametrize("kind", ["full", "chain", "binary"])
def test_tree_attention_oracle_vs_sdpa(kind):
    g = torch.Generator().manual_seed(2)
    B, N, Hq, Hkv, D, bs = 2, 15, 4, 2, 16, 8
    ctx = [21, 8]
    if kind == "full":
        masks = np.array([(1 << N) - 1] * N, dtype=np.uint64)
    elif kind == "chain":
        masks = T.ancestor_masks(T.chain_parents(N))
    else:
        masks = T.ancestor_masks(T.binary_tree_parents(N))
    K = [torch.randn(c + N, Hkv, D, generator=g) for c in ctx]
    V = [torch.randn(c + N, Hkv, D, generator=g) for c in ctx]
    kp, vp, bt = H.paged_pools(K, V, block_size=bs)
    q = torch.randn(B, N, Hq, D, generator=g)
    scale = D ** -0.5
    got = O.tree_attention(q, kp, vp, bt, ctx, 0, masks, bs, scale)
    for b in range(B):
        L = ctx[b] + N
        allow = torch.ones(N, L, dtype=torch.bool)
        for i in range(N):
            for j in range(N):
                allow[i, ctx[b] + j] = bool((int(masks[i]) >> j) & 1)
        if kind == "chain":  # the chain tree is causal attention over ctx + N
            causal = torch.ones(N, L, dtype=torch.bool).tril(diagonal=ctx[b])
            assert torch.equal(allow, causal)
        want = _ref_sdpa(q[b], K[b], V[b], allow, scale)
        assert (got[b].double() - want).abs().max() < 1e-5


def test_kv_commit_oracle_vs_index_copy():
    g = torch.Generator().manual_seed(3)
    B, N, Hkv, D, bs, layers = 3, 15, 2, 8, 4, 2
    ctx = [9, 4, 16]
    K = [torch.randn(c + N, Hkv, D, generator=g) for c in ctx]
    kp, vp, bt = H.paged_pools(K, K, block_size=bs, num_layers=layers)
    paths = [[0, 1, 3, 7], [0, 2], [0]]
    lens = [len(p) for p in paths]
    k2, v2, new_lens = O.kv_commit(kp, vp, bt, ctx, [p + [0] * (4 - len(p)) for p in paths],
                                   lens, bs)
    assert list(new_lens) == [c + n for c, n in zip(ctx, lens)]
    for b in range(B):
        for layer in range(layers):
            before = O.gather_pages(kp, bt[b], ctx[b] + N, layer, bs)
            after = O.gather_pages(k2, bt[b], ctx[b] + N, layer, bs)
            src = torch.tensor([ctx[b] + j for j in paths[b]])
            want = before.clone().index_copy(0, torch.arange(ctx[b], ctx[b] + lens[b]),
                                             before[src])
            assert torch.equal(after, want)


# --- tree acceptance oracle (orc_tree_verify) -------------------------------


def test_tree_walk_on_chain_equals_chain_verify():
    """On a one-child chain the tree walk is verify_candidates
    (speculative.cpp:50-103): same accept count, final token and EOS."""
    from tests.golden.recipes import chain_case

    for seed in range(6):
        K, V = 5, 300
        tok, d, t, eos = chain_case(500 + seed, 4, K, V, eos_bias=(seed % 2 == 0))
        U = np.random.default_rng(seed).random((4, K + 1)).astype(np.float32)
        want = O.chain_verify(t, d, tok, U, eos=eos)
        parents = T.chain_parents(K + 1)
        for c in range(4):
            ntok = np.concatenate([[0], tok[c]]).astype(np.int32)
            dd = np.concatenate([d[c], np.zeros((1, V), np.float32)])
            w = O.tree_verify(parents, ntok, t[c], dd, U[c], eos=eos)
            assert len(w["path"]) - 1 == want["accept_len"][c]
            assert w["final"] == want["final"][c] and int(w["eos"]) == want["eos"][c]


def test_tree_walk_preserves_target_distribution():
    """Multi-candidate rejection sampling emits its first token with exactly
    the target distribution p_root when the candidates are drawn from the
    draft distribution q (SpecInfer, Miao et al. 2023): chi-square test on a
    3-candidate star over V = 5."""
    rng = np.random.default_rng(123)
    V, n = 5, 40000
    p = np.array([0.05, 0.4, 0.1, 0.25, 0.2], np.float32)
    q = np.array([0.3, 0.1, 0.3, 0.2, 0.1], np.float32)
    parents = np.array([-1, 0, 0, 0], np.int32)
    tp = np.stack([p, p, p, p])           # rows of the leaves are never sampled here
    dp = np.stack([q, q, q, q])
    counts = np.zeros(V)
    cq = np.cumsum(q.astype(np.float64))
    for _ in range(n):
        toks = [0] + [int(np.searchsorted(cq, rng.random() * cq[-1])) for _ in range(3)]
        U = rng.random(8).astype(np.float32)
        w = O.tree_verify(parents, np.array(toks, np.int32), tp, dp, U)
        first = toks[w["path"][1]] if len(w["path"]) > 1 else w["final"]
        counts[first] += 1
    expected = n * p.astype(np.float64)
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 18.47, (chi2, counts / n)  # chi-square(4) 99.9% quantile


def test_tree_walk_greedy_known_answer():
    # root's argmax is token 2; children carry tokens 1 and 2 -> node 2 accepted;
    # node 2 is a leaf whose argmax (token 3) is the bonus
    parents = np.array([-1, 0, 0], np.int32)
    tp = np.array([[0.1, 0.2, 0.6, 0.1], [0.25] * 4, [0.1, 0.1, 0.1, 0.7]], np.float32)
    w = O.tree_verify(parents, np.array([0, 1, 2], np.int32), tp, tp, np.zeros(1, np.float32),
                      greedy=True)
    assert list(w["path"]) == [0, 2] and w["final"] == 3
