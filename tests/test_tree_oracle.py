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
