"""GPU tier: tree-masked paged attention (cfa_tree_attention) against the fp32
oracle (masked SDPA over pages gathered on the CPU), tolerance 1e-2 abs."""
import numpy as np
import pytest
import torch

from cudaforge_amd import tree as T
from cudaforge_amd.verify import tree_attention
from oracle import oracle as O
from tests import helpers as H

pytestmark = pytest.mark.gpu

ATOL = 1e-2  # bf16 inputs and output, fp32 softmax / accumulation


def _case(B, N, Hq, Hkv, ctx, bs, parents, per_seq_masks=False, layers=1, layer=0, seed=0, D=128):
    g = torch.Generator().manual_seed(seed)
    K = [torch.randn(c + N, Hkv, D, generator=g).bfloat16() for c in ctx]
    V = [torch.randn(c + N, Hkv, D, generator=g).bfloat16() for c in ctx]
    kp, vp, bt = H.paged_pools(K, V, block_size=bs, num_layers=layers, layer=layer, seed=seed)
    q = torch.randn(B, N, Hq, D, generator=g).bfloat16()
    if per_seq_masks:
        masks = np.stack([T.ancestor_masks(parents(b)) for b in range(B)])
    else:
        masks = T.ancestor_masks(parents(0))
    return q, kp, vp, bt, masks


def _run(device, q, kp, vp, bt, ctx, masks, bs, layer=0, splits=0, first_node=0):
    N = q.shape[1]
    mt = T.mask_tensor(masks, device)
    out = tree_attention(q[:, first_node:].to(device), kp.to(device), vp.to(device), bt.to(device),
                         torch.tensor(ctx, dtype=torch.int32, device=device), mt, layer=layer,
                         max_keys=max(ctx) + N, num_splits=splits, first_node=first_node)
    torch.cuda.synchronize()
    return out.float().cpu()


def _oracle(q, kp, vp, bt, ctx, masks, bs, layer=0):
    scale = q.shape[-1] ** -0.5
    if masks.ndim == 1:
        return O.tree_attention(q, kp, vp, bt, ctx, layer, masks, bs, scale)
    outs = [O.tree_attention(q[b:b + 1], kp, vp, bt[b:b + 1], ctx[b:b + 1], layer, masks[b], bs,
                             scale) for b in range(q.shape[0])]
    return torch.cat(outs)


@pytest.mark.parametrize("splits", [1, 2, 0])
def test_small_binary_tree(device, splits):
    B, N, Hq, Hkv, bs = 3, 15, 8, 2, 16
    ctx = [100, 37, 256]
    q, kp, vp, bt, masks = _case(B, N, Hq, Hkv, ctx, bs, lambda b: T.binary_tree_parents(N))
    got = _run(device, q, kp, vp, bt, ctx, masks, bs, splits=splits)
    want = _oracle(q, kp, vp, bt, ctx, masks, bs)
    err = (got - want).abs().max().item()
    assert err <= ATOL, err


def test_per_sequence_trees_block32_layer1(device):
    B, N, Hq, Hkv, bs = 4, 31, 4, 4, 32
    ctx = [1, 64, 200, 333]
    rng = np.random.default_rng(5)

    def parents(b):
        p = [-1] + [int(rng.integers(0, i)) for i in range(1, N)]
        return np.array(p, np.int32)

    q, kp, vp, bt, masks = _case(B, N, Hq, Hkv, ctx, bs, parents, per_seq_masks=True, layers=3,
                                 layer=1, seed=4)
    got = _run(device, q, kp, vp, bt, ctx, masks, bs, layer=1)
    want = _oracle(q, kp, vp, bt, ctx, masks, bs, layer=1)
    err = (got - want).abs().max().item()
    assert err <= ATOL, err


def test_chain_tree_is_causal_attention(device):
    B, N, Hq, Hkv, bs = 2, 9, 32, 8, 16
    ctx = [77, 130]
    q, kp, vp, bt, masks = _case(B, N, Hq, Hkv, ctx, bs, lambda b: T.chain_parents(N), seed=7)
    got = _run(device, q, kp, vp, bt, ctx, masks, bs)
    want = _oracle(q, kp, vp, bt, ctx, masks, bs)
    assert (got - want).abs().max().item() <= ATOL


def test_c3_shape(device):
    """B=16, 63-node binary tree, 32 q / 8 KV heads,
    head_dim 128, context 4096, page 16, random page table."""
    B, N, Hq, Hkv, bs, C = 16, 63, 32, 8, 16, 4096
    ctx = [C] * B
    q, kp, vp, bt, masks = _case(B, N, Hq, Hkv, ctx, bs, lambda b: T.binary_tree_parents(N),
                                 seed=11)
    got = _run(device, q, kp, vp, bt, ctx, masks, bs)
    want = _oracle(q, kp, vp, bt, ctx, masks, bs)
    err = (got - want).abs().max().item()
    assert err <= ATOL, err
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("splits", [1, 3, 0])
def test_head_dim_64(device, splits):
    B, N, Hq, Hkv, bs = 3, 15, 8, 2, 16
    ctx = [100, 37, 300]
    q, kp, vp, bt, masks = _case(B, N, Hq, Hkv, ctx, bs, lambda b: T.binary_tree_parents(N),
                                 seed=21, D=64)
    got = _run(device, q, kp, vp, bt, ctx, masks, bs, splits=splits)
    want = _oracle(q, kp, vp, bt, ctx, masks, bs)
    err = (got - want).abs().max().item()
    assert err <= ATOL, err


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("first_node", [1, 7, 14])
def test_first_node_queries_a_suffix(device, D, first_node):
    """Queries of nodes first_node..N-1 only: the rows of the full call."""
    B, N, Hq, Hkv, bs = 2, 15, 8, 2, 16
    ctx = [64, 129]
    rng = np.random.default_rng(first_node)

    def parents(b):
        return np.array([-1] + [int(rng.integers(0, i)) for i in range(1, N)], np.int32)

    q, kp, vp, bt, masks = _case(B, N, Hq, Hkv, ctx, bs, parents, per_seq_masks=True, seed=3, D=D)
    got = _run(device, q, kp, vp, bt, ctx, masks, bs, first_node=first_node)
    want = _oracle(q, kp, vp, bt, ctx, masks, bs)[:, first_node:]
    assert got.shape == want.shape
    err = (got - want).abs().max().item()
    assert err <= ATOL, err


def test_draft_level_shape(device):
    """A 1B-shape draft growing a binary tree: level 4 (nodes 15..30) of 31
    nodes, head_dim 64, 32 / 8 heads, B = 8, context 2048."""
    B, N, Hq, Hkv, bs, C = 8, 31, 32, 8, 16, 2048
    ctx = [C + 3 * b for b in range(B)]
    q, kp, vp, bt, masks = _case(B, N, Hq, Hkv, ctx, bs, lambda b: T.binary_tree_parents(N),
                                 seed=13, D=64)
    got = _run(device, q, kp, vp, bt, ctx, masks, bs, first_node=15)
    want = _oracle(q, kp, vp, bt, ctx, masks, bs)[:, 15:]
    err = (got - want).abs().max().item()
    assert err <= ATOL, err
    assert torch.isfinite(got).all()
