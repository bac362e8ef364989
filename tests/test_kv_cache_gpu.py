"""GPU tier: the paged KV cache's device side -- batch metadata staged into
device buffers (the reference's own test, tests/cpp/test_paged_kv_cache.cpp:
38-80), copy on write of a page shared after fork, and the commit + rollback
of an accepted draft-tree path through the cache (cfa_kv_commit + truncate)
against the oracle (oracle/oracle.py kv_commit; oracle/kv_pages.py tables).
Bit-exact."""
import numpy as np
import pytest
import torch

from cudaforge_amd import tree as T
from cudaforge_amd.kv_cache import KVCacheConfig, PagedKVCache
from oracle import oracle as O
from oracle.kv_pages import PageTables

pytestmark = pytest.mark.gpu


def test_reference_kat_on_device(device):
    cfg = KVCacheConfig(num_layers=2, num_kv_heads=2, head_dim=64, block_size=16,
                        element_size_bytes=2, total_gpu_blocks=32, max_supported_batch_size=16,
                        max_blocks_per_sequence=32)
    kv = PagedKVCache(cfg, device=device)
    kv.register_sequence_with_prefix(100, [1] * 32)
    kv.register_sequence_with_prefix(200, [2] * 48)
    stream = torch.cuda.Stream(device)
    d = kv.prepare_batch_metadata([100, 200], stream=stream)
    stream.synchronize()
    assert d.batch_size == 2 and d.max_blocks_per_seq == 3
    assert d.block_tables.device.type == "cuda" and d.context_lens.device.type == "cuda"
    assert d.key_pool_ptr != 0 and d.val_pool_ptr != 0
    assert d.context_lens.cpu().tolist() == [32, 48]
    assert d.block_tables.cpu().tolist() == [[0, 1, -1], [2, 3, 4]]
    assert kv.key_pool.dtype == torch.bfloat16
    assert kv.get_key_block_ptr(3, 1) == kv.key_pool[3, 1].data_ptr()
    assert kv.get_value_block_ptr(5, 0) == kv.value_pool[5, 0].data_ptr()
    # a second call reuses the staging buffers (stream ordered)
    kv.append_tokens(100, 1)
    d2 = kv.prepare_batch_metadata([200, 100])
    torch.cuda.synchronize()
    assert d2.context_lens.cpu().tolist() == [48, 33]
    assert d2.block_tables.cpu().tolist() == [[2, 3, 4], [0, 1, 5]]
    kv.unregister_sequence(100)
    kv.unregister_sequence(200)


def test_copy_on_write_copies_pool_rows(device):
    cfg = KVCacheConfig(num_layers=3, num_kv_heads=2, head_dim=128, block_size=16,
                        total_gpu_blocks=8, max_supported_batch_size=4, max_blocks_per_sequence=8)
    kv = PagedKVCache(cfg, device=device)
    g = torch.Generator().manual_seed(1)
    kv.key_pool.copy_(torch.randn(kv.key_pool.shape, generator=g).bfloat16())
    kv.value_pool.copy_(torch.randn(kv.value_pool.shape, generator=g).bfloat16())
    k0, v0 = kv.key_pool.clone(), kv.value_pool.clone()
    kv.register_sequence_with_prefix(1, list(range(21)))     # [0 hashed, 1 with 5 tokens]
    kv.fork_sequence(1, 2)
    kv.append_tokens(2, 3)                                   # child: private copy of page 1
    assert kv.get_block_table(2) == [0, 2] and kv.get_block_table(1) == [0, 1]
    torch.cuda.synchronize()
    assert torch.equal(kv.key_pool[2, :, :, :5], k0[1, :, :, :5])
    assert torch.equal(kv.value_pool[2, :, :, :5], v0[1, :, :, :5])
    assert torch.equal(kv.key_pool[2, :, :, 5:], k0[2, :, :, 5:])    # rest untouched
    assert torch.equal(kv.key_pool[1], k0[1]) and torch.equal(kv.value_pool[1], v0[1])


@pytest.mark.parametrize("bs,N", [(16, 15), (32, 31)])
def test_tree_commit_and_rollback_through_cache(device, bs, N):
    rng = np.random.default_rng(bs + N)
    Hkv, D, layers = 2, 128, 2
    cfg = KVCacheConfig(num_layers=layers, num_kv_heads=Hkv, head_dim=D, block_size=bs,
                        total_gpu_blocks=64, max_supported_batch_size=8, max_blocks_per_sequence=16)
    kv = PagedKVCache(cfg, device=device)
    orc = PageTables(num_blocks=64, block_size=bs, max_batch=8, max_blocks_per_seq=16)
    g = torch.Generator().manual_seed(bs)
    kv.key_pool.copy_(torch.randn(kv.key_pool.shape, generator=g).bfloat16())
    kv.value_pool.copy_(torch.randn(kv.value_pool.shape, generator=g).bfloat16())
    seqs = [11, 12, 13, 14]
    prompts = [list(rng.integers(0, 50, int(n))) for n in (5, bs, 2 * bs + 3, 40)]
    prompts[3][:bs] = prompts[1]           # shares its first page with sequence 12
    for s, p in zip(seqs, prompts):
        assert kv.register_sequence_with_prefix(s, p) == orc.register(s, p)
    base = [kv.context_length(s) for s in seqs]
    for s in seqs:                          # slots for the N tree nodes
        kv.append_tokens(s, N)
        orc.append(s, N)
    d = kv.prepare_batch_metadata(seqs)
    parents = T.binary_tree_parents(N)
    paths = np.zeros((len(seqs), 6), np.int32)
    lens = np.zeros(len(seqs), np.int32)
    for b in range(len(seqs)):
        node = int(rng.integers(0, N))
        chain = [node]
        while parents[chain[-1]] >= 0:
            chain.append(int(parents[chain[-1]]))
        chain = chain[::-1][:6]
        paths[b, :len(chain)] = chain
        lens[b] = len(chain)
    tables, _, _ = orc.prepare_batch(seqs)
    want_k, want_v, want_len = O.kv_commit(kv.key_pool.cpu(), kv.value_pool.cpu(),
                                           torch.tensor(tables, dtype=torch.int32), base,
                                           paths, lens, bs)
    new_lens = kv.commit_tree_paths(seqs, d, torch.tensor(base, dtype=torch.int32, device=device),
                                    torch.from_numpy(paths).to(device),
                                    torch.from_numpy(lens).to(device))
    torch.cuda.synchronize()
    assert new_lens == list(want_len)
    assert torch.equal(kv.key_pool.cpu(), want_k) and torch.equal(kv.value_pool.cpu(), want_v)
    for s, n in zip(seqs, new_lens):
        orc.truncate(s, n)
        assert kv.context_length(s) == n
        assert kv.get_block_table(s) == orc.tables[s]
    st, so = vars(kv.get_stats()), orc.stats()
    for k in ("free_blocks", "cached_prefix_blocks", "allocated_blocks"):
        assert st[k] == so[k]
