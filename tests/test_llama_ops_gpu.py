"""GPU tier: the fused layers of the model-scale step (cfa_rmsnorm,
cfa_rope_kv_paged / _strided, cfa_silu_mul) against PyTorch restatements of
the same formulas.  Tolerances are stated per test: one bf16 rounding step
(2^-8 relative) where only the fp32 reduction order or the exp / sincos
implementation differs."""
import math

import pytest
import torch

from cudaforge_amd.kv_cache import KVCacheConfig, PagedKVCache
from cudaforge_amd.spec_step import LlamaShape, rmsnorm_, rope_kv_paged, rope_kv_strided, silu_mul

pytestmark = pytest.mark.gpu

ULP = 2.0 ** -8


def _rope_ref(x, pos, theta):
    D = x.shape[-1]
    inv = theta ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = pos.double()[:, None] * inv
    cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]
    xf = x.double()
    rot = torch.cat([-xf[..., D // 2:], xf[..., : D // 2]], -1)
    return xf * cos + rot * sin


@pytest.mark.parametrize("with_delta", [False, True])
def test_rmsnorm(device, with_delta):
    M, d = 37, 4096
    g = torch.Generator().manual_seed(1)
    h = torch.randn(M, d, generator=g).bfloat16()
    delta = torch.randn(M, d, generator=g).bfloat16() if with_delta else None
    w = (1 + 0.1 * torch.randn(d, generator=g)).bfloat16()
    hd = h.to(device)
    out = torch.empty_like(hd)
    rmsnorm_(hd, delta.to(device) if with_delta else None, w.to(device), 1e-5, out)
    hh = (h + delta) if with_delta else h                 # bf16 add, as PyTorch rounds it
    assert torch.equal(hd.cpu(), hh)
    xf = hh.double()
    ref = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.double()
    err = ((out.cpu().double() - ref).abs() / ref.abs().clamp_min(1e-3)).max().item()
    assert err <= 2 * ULP, err


def test_silu_mul(device):
    M, F = 19, 3000
    gu = (3 * torch.randn(M, 2 * F, generator=torch.Generator().manual_seed(2))).bfloat16()
    out = silu_mul(gu.to(device)).cpu().double()
    g, u = gu[:, :F].double(), gu[:, F:].double()
    ref = g / (1 + torch.exp(-g)) * u
    err = ((out - ref).abs() / ref.abs().clamp_min(1e-2)).max().item()
    assert err <= 2 * ULP, err


def test_silu_mul_vector_path_bit_exact(device):
    """The 8-wide kernel (F % 8 == 0, aligned) and the one-element kernel
    (taken here through a 2-byte-misaligned output) give identical bits."""
    from cudaforge_amd import _lib
    from cudaforge_amd.verify import _stream_ptr

    M, F = 7, 4096
    gu = (3 * torch.randn(M, 2 * F, generator=torch.Generator().manual_seed(5))).bfloat16().to(device)
    buf = torch.empty(2 * M * F + 16, dtype=torch.bfloat16, device=device)
    aligned = buf[: M * F]
    shifted = buf[M * F + 1: 2 * M * F + 1]
    lib = _lib.load()
    for out in (aligned, shifted):
        _lib.check(lib.cfa_silu_mul(gu.data_ptr(), out.data_ptr(), M, F, _stream_ptr(gu.device)),
                   "cfa_silu_mul")
    torch.cuda.synchronize()
    assert shifted.data_ptr() % 16 != 0
    assert torch.equal(aligned.view(torch.int16), shifted.view(torch.int16))


def test_rope_kv_paged(device):
    s = LlamaShape(2, 512, 4, 2, 128, 256, 100)
    B, n, bs = 3, 5, 16
    cfg = KVCacheConfig(num_layers=2, num_kv_heads=2, head_dim=128, block_size=bs,
                        total_gpu_blocks=32, max_supported_batch_size=4, max_blocks_per_sequence=8)
    kv = PagedKVCache(cfg, device=device)
    kv.key_pool.zero_()
    kv.value_pool.zero_()
    ctx = [13, 30, 0]
    for b in range(B):
        kv.register_sequence_with_prefix(b, list(range(ctx[b])))
        kv.append_tokens(b, n)
    desc = kv.prepare_batch_metadata(list(range(B)))
    H = s.n_heads + 2 * s.n_kv_heads
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(B * n, H * 128, generator=g).bfloat16()
    pos = torch.tensor([c + j * 7 for c in ctx for j in range(n)], dtype=torch.int32)
    q = torch.empty(B * n, s.n_heads, 128, dtype=torch.bfloat16, device=device)
    base = torch.tensor(ctx, dtype=torch.int32, device=device)
    rope_kv_paged(qkv.to(device), pos.to(device), B, n, s, q, kv, 1, desc.block_tables, base)
    torch.cuda.synchronize()
    x = qkv.view(B * n, H, 128)
    ref = _rope_ref(x[:, : s.n_heads + s.n_kv_heads], pos, s.rope_theta)
    assert (q.cpu().double() - ref[:, : s.n_heads]).abs().max().item() <= 2 * ULP * ref.abs().max()
    tables = desc.block_tables.cpu()
    kp, vp = kv.key_pool.cpu(), kv.value_pool.cpu()
    for b in range(B):
        for j in range(n):
            slot = ctx[b] + j
            blk = int(tables[b, slot // bs])
            m = b * n + j
            kref = ref[m, s.n_heads:]
            assert (kp[blk, 1, :, slot % bs].double() - kref).abs().max() <= 2 * ULP * kref.abs().max()
            assert torch.equal(vp[blk, 1, :, slot % bs], x[m, s.n_heads + s.n_kv_heads:])
            assert not kp[blk, 0, :, slot % bs].any()            # other layer untouched


@pytest.mark.parametrize("splits", [1, 3, 5])
def test_rope_kv_paged_partials_bit_exact(device, splits):
    """cfa_rope_kv_paged_partials on fp32 split-K partials [S, M, H*D] gives
    the bits of cfa_rope_kv_paged on bf16 of their sum in slab order (what
    the W4A16 GEMM's reduce writes): q, the K/V pools, and the untouched
    layer."""
    s = LlamaShape(2, 512, 4, 2, 128, 256, 100)
    B, n, bs = 3, 5, 16
    H = s.n_heads + 2 * s.n_kv_heads
    g = torch.Generator().manual_seed(11 + splits)
    part = torch.randn(splits, B * n, H * 128, generator=g).to(device)
    acc = part[0].clone()
    for i in range(1, splits):
        acc += part[i]                                   # fp32, slab order
    qkv = acc.bfloat16()
    pos = torch.tensor([c + j * 7 for c in (13, 30, 0) for j in range(n)], dtype=torch.int32,
                       device=device)
    outs = []
    for src in (part, qkv):
        cfg = KVCacheConfig(num_layers=2, num_kv_heads=2, head_dim=128, block_size=bs,
                            total_gpu_blocks=32, max_supported_batch_size=4,
                            max_blocks_per_sequence=8)
        kv = PagedKVCache(cfg, device=device)
        kv.key_pool.zero_()
        kv.value_pool.zero_()
        for b, c in enumerate((13, 30, 0)):
            kv.register_sequence_with_prefix(b, list(range(c)))
            kv.append_tokens(b, n)
        desc = kv.prepare_batch_metadata(list(range(B)))
        q = torch.empty(B * n, s.n_heads, 128, dtype=torch.bfloat16, device=device)
        base = torch.tensor([13, 30, 0], dtype=torch.int32, device=device)
        rope_kv_paged(src, pos, B, n, s, q, kv, 1, desc.block_tables, base)
        outs.append((q, kv.key_pool.clone(), kv.value_pool.clone()))
    torch.cuda.synchronize()
    for x, y in zip(*outs):
        assert torch.equal(x, y)


def test_rope_kv_strided(device):
    s = LlamaShape(1, 256, 4, 2, 64, 256, 100)
    B, n, S = 2, 3, 40
    H = s.n_heads + 2 * s.n_kv_heads
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(B * n, H * 64, generator=g).bfloat16()
    pos = torch.randint(0, 1000, (B * n,), generator=g, dtype=torch.int32)
    slots = torch.tensor([[5, 9, 33], [0, 1, 39]], dtype=torch.int32)
    kT = torch.zeros(B, s.n_kv_heads, 64, S, dtype=torch.bfloat16, device=device)
    v = torch.zeros(B, s.n_kv_heads, S, 64, dtype=torch.bfloat16, device=device)
    q = torch.empty(B * n, s.n_heads, 64, dtype=torch.bfloat16, device=device)
    rope_kv_strided(qkv.to(device), pos.to(device), B, n, s, q, kT, v, slots.to(device))
    torch.cuda.synchronize()
    x = qkv.view(B * n, H, 64)
    ref = _rope_ref(x[:, : s.n_heads + s.n_kv_heads], pos, s.rope_theta)
    tol = 2 * ULP * ref.abs().max()
    assert (q.cpu().double() - ref[:, : s.n_heads]).abs().max() <= tol
    kc, vc = kT.cpu(), v.cpu()
    for b in range(B):
        for j in range(n):
            m, sl = b * n + j, int(slots[b, j])
            assert (kc[b, :, :, sl].double() - ref[m, s.n_heads:]).abs().max() <= tol
            assert torch.equal(vc[b, :, sl], x[m, s.n_heads + s.n_kv_heads:])
