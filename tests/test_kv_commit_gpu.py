"""GPU tier: KV commit / compaction (cfa_kv_commit) against the oracle
(index_copy of accepted slots over gathered pages) -- bit-exact."""
import numpy as np
import pytest
import torch

from cudaforge_amd import tree as T
from cudaforge_amd.verify import kv_commit
from oracle import oracle as O
from tests import helpers as H

pytestmark = pytest.mark.gpu


def _random_paths(rng, parents, B, maxlen):
    """Root-to-node paths of random lengths (root first)."""
    N = len(parents)
    paths = np.zeros((B, maxlen), np.int32)
    lens = np.zeros(B, np.int32)
    for b in range(B):
        node = int(rng.integers(0, N))
        chain = [node]
        while parents[chain[-1]] >= 0:
            chain.append(int(parents[chain[-1]]))
        chain = chain[::-1][:maxlen]
        paths[b, : len(chain)] = chain
        lens[b] = len(chain)
    return paths, lens


@pytest.mark.parametrize("layers,bs", [(32, 16), (4, 16), (2, 32)])
def test_commit_matches_oracle(device, layers, bs):
    """(32, 16) is the full tree-commit shape: B = 32, 63-node tree, 32 layers
    x 8 KV heads x 128, pages of 16."""
    rng = np.random.default_rng(layers * 10 + bs)
    B, N, Hkv, D = 32, 63, 8, 128
    parents = T.binary_tree_parents(N)
    ctx = [int(x) for x in rng.integers(1, 300, B)]
    g = torch.Generator().manual_seed(3)
    K = [torch.randn(c + N, Hkv, D, generator=g).bfloat16() for c in ctx]
    kp, vp, bt = H.paged_pools(K, K, block_size=bs, num_layers=layers, layer=0, seed=5)
    paths, lens = _random_paths(rng, parents, B, 7)
    want_k, want_v, want_len = O.kv_commit(kp, vp, bt, ctx, paths, lens, bs)
    kd, vd = kp.to(device), vp.to(device)
    out = kv_commit(kd, vd, bt.to(device), torch.tensor(ctx, dtype=torch.int32, device=device),
                    torch.from_numpy(paths).to(device), torch.from_numpy(lens).to(device))
    torch.cuda.synchronize()
    assert out.status.cpu().tolist() == [0] * B
    assert out.new_ctx_lens.cpu().tolist() == list(want_len)
    assert torch.equal(kd.cpu(), want_k)
    assert torch.equal(vd.cpu(), want_v)


def test_commit_rejects_bad_paths_and_keeps_pools(device):
    B, N, Hkv, D, bs = 3, 15, 2, 128, 16
    ctx = [20, 5, 40]
    g = torch.Generator().manual_seed(9)
    K = [torch.randn(c + N, Hkv, D, generator=g).bfloat16() for c in ctx]
    kp, vp, bt = H.paged_pools(K, K, block_size=bs, num_layers=1)
    paths = np.array([[0, 2, 1, 0], [1, 3, 0, 0], [0, 1, 3, 7]], np.int32)  # bad, bad, good
    lens = np.array([3, 2, 4], np.int32)
    kd, vd = kp.to(device), vp.to(device)
    out = kv_commit(kd, vd, bt.to(device), torch.tensor(ctx, dtype=torch.int32, device=device),
                    torch.from_numpy(paths).to(device), torch.from_numpy(lens).to(device))
    torch.cuda.synchronize()
    assert out.status.cpu().tolist() == [1, 1, 0]
    assert out.new_ctx_lens.cpu().tolist() == [20, 5, 44]
    want_k, want_v, _ = O.kv_commit(kp, vp, bt, ctx, [[0], [0], [0, 1, 3, 7]], [1, 1, 4], bs)
    assert torch.equal(kd.cpu(), want_k) and torch.equal(vd.cpu(), want_v)


def test_full_chain_acceptance_is_noop(device):
    B, N, Hkv, D, bs = 2, 9, 2, 128, 16
    ctx = [16, 33]
    g = torch.Generator().manual_seed(1)
    K = [torch.randn(c + N, Hkv, D, generator=g).bfloat16() for c in ctx]
    kp, vp, bt = H.paged_pools(K, K, block_size=bs, num_layers=2)
    paths = np.tile(np.arange(N, dtype=np.int32), (B, 1))
    lens = np.full(B, N, np.int32)
    kd, vd = kp.to(device), vp.to(device)
    out = kv_commit(kd, vd, bt.to(device), torch.tensor(ctx, dtype=torch.int32, device=device),
                    torch.from_numpy(paths).to(device), torch.from_numpy(lens).to(device))
    torch.cuda.synchronize()
    assert out.new_ctx_lens.cpu().tolist() == [c + N for c in ctx]
    assert torch.equal(kd.cpu(), kp) and torch.equal(vd.cpu(), vp)
