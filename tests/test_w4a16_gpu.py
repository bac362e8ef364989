"""GPU tier: W4A16 dequantisation (cfa_w4a16_dequant, and its transposed
output cfa_w4a16_dequant_t) bit-exact against a
numpy restatement of the reference formula (int4_gemm_dequant.cu:20-31,
int4_dequant_triton.py:74-78), and the reference's own GEMM parity test
(tests/unit/test_int4_dequant.py:18-53: atol = rtol = 1e-2 against an fp16
dequantised matmul)."""
import numpy as np
import pytest
import torch

from cudaforge_amd.w4a16 import int4_gemm_dequant, pack_int4_weights, w4a16_dequant

pytestmark = pytest.mark.gpu


def _np_dequant(w_int4, scales, zeros, group, dtype):
    """fp16: (fp16(n) - z) * s with each operation rounded to fp16 (the fp32
    result of a difference or product of these fp16 operands is exact, so one
    rounding to fp16 is the correctly rounded fp16 operation); bf16: the fp32
    value (n - z) * s rounded to nearest even."""
    K, N = w_int4.shape
    g = np.arange(K) // group
    s = scales[g].astype(np.float32)
    n = w_int4.astype(np.float32)
    if dtype == "fp16":
        z = zeros[g].astype(np.float32) if zeros is not None else np.zeros_like(s)
        d = (n - z).astype(np.float16).astype(np.float32)
        return (d * s).astype(np.float16)
    z = zeros[g].astype(np.float32) if zeros is not None else 0.0
    f = ((n - z) * s).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("with_zeros", [False, True])
@pytest.mark.parametrize("K,N,group", [(128, 256, 128), (512, 96, 64), (1024, 48, 128),
                                       (256, 50, 128), (136, 300, 8)])
@pytest.mark.parametrize("transposed", [False, True])
def test_dequant_bit_exact(device, dtype, with_zeros, K, N, group, transposed):
    """Both output layouts: [K, N] (cfa_w4a16_dequant) and [N, K]
    (cfa_w4a16_dequant_t, 16 packed rows per thread: K = 136 leaves a tail)."""
    g = torch.Generator().manual_seed(K + N)
    w = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    scales = (torch.rand(K // group, N, generator=g) * 0.1 + 1e-3).half()
    zeros = torch.randint(0, 16, (K // group, N), generator=g).half() if with_zeros else None
    q = pack_int4_weights(w)
    out = w4a16_dequant(q.to(device), scales.to(device),
                        zeros.to(device) if zeros is not None else None, group_size=group,
                        dtype=torch.float16 if dtype == "fp16" else torch.bfloat16,
                        transposed=transposed)
    want = _np_dequant(w.numpy(), scales.numpy(), zeros.numpy() if zeros is not None else None,
                       group, dtype)
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    exp = want.view(np.uint16)
    if transposed:
        exp = np.ascontiguousarray(exp.T)
    assert np.array_equal(got, exp)


def test_pack_layout_known_answer():
    w = torch.arange(16, dtype=torch.int32).reshape(16, 1) % 16
    q = pack_int4_weights(w)
    assert q.shape == (2, 1)
    assert q[0, 0].item() == 0x76543210
    assert q[1, 0].item() == np.int32(np.uint32(0xFEDCBA98)).item()


@pytest.mark.parametrize("M", [16, 64])
@pytest.mark.parametrize("N", [128, 256])
@pytest.mark.parametrize("K", [128, 512])
def test_reference_gemm_parity(device, M, N, K):
    group = 128
    torch.manual_seed(42)
    a = torch.randn((M, K), dtype=torch.float16, device=device)
    w_int4 = torch.randint(0, 16, (K, N), device=device, dtype=torch.int32)
    scales = torch.randn((K // group, N), dtype=torch.float16, device=device).abs() * 0.1
    b_quant = pack_int4_weights(w_int4)
    w_dequant = torch.zeros((K, N), dtype=torch.float16, device=device)
    for k in range(K):
        w_dequant[k, :] = w_int4[k, :].to(torch.float16) * scales[k // group, :]
    c_ref = torch.matmul(a, w_dequant)
    c = int4_gemm_dequant(a, b_quant, scales, group_size=group)
    torch.testing.assert_close(c, c_ref, atol=1e-2, rtol=1e-2)


_FUSED_SHAPES = [(1, 256, 128), (37, 1024, 512), (504, 512, 4096), (64, 768, 256),
                 (200, 256, 1024), (504, 8192, 256), (504, 28672, 128), (504, 6144, 256)]


@pytest.mark.parametrize("dtype,M,N,K",
                         [(d, *shape) for d in (torch.bfloat16, torch.float16) for shape in _FUSED_SHAPES]
                         + [(torch.bfloat16, 130, 192, 512)])
def test_fused_gemm_vs_dequantised_fp32(device, dtype, M, N, K):
    """cfa_w4a16_gemm against an fp32 product of the bit-exact dequantised
    weights: differences come from the fp32 accumulation order and the final
    rounding to 16 bits (tolerance 1e-2 of the output scale + 2^-7 relative).
    bf16 with M > 64 takes the cooperative-dequantisation kernel: 64-column
    tiles at (504, 512), (200, 256), (130, 192: a partial last m-tile; bf16
    only, as the fp16 kernel takes N % 256 == 0), 128-column tiles at
    (504, 8192); grids of at most one work-group per CU use the 5-stage
    ring, (504, 28672) and (504, 6144) the 3-stage one at 128 and 64
    columns."""
    from cudaforge_amd.w4a16 import w4a16_gemm

    g = torch.Generator().manual_seed(M + N + K)
    group = 128
    a = torch.randn(M, K, generator=g).to(dtype).to(device)
    w_int4 = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    scales = (torch.rand(K // group, N, generator=g) * 0.05 + 1e-3).half().to(device)
    q = pack_int4_weights(w_int4).to(device)
    c = w4a16_gemm(a, q, scales, group_size=group)
    w = w4a16_dequant(q, scales, group_size=group, dtype=dtype).float()
    ref = a.float() @ w
    torch.cuda.synchronize()
    err = (c.float() - ref).abs()
    tol = 1e-2 * ref.abs().max() + 2.0 ** -7 * ref.abs()
    assert (err <= tol).all(), err.max().item()


def test_fused_gemm_rejects_bad_shapes(device):
    from cudaforge_amd.w4a16 import w4a16_gemm

    a = torch.randn(4, 128, device=device).bfloat16()
    q = torch.zeros(16, 100, dtype=torch.int32, device=device)
    s = torch.ones(1, 100, dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        w4a16_gemm(a, q, s)


@pytest.mark.parametrize("K,N,with_zeros", [(4096, 8192, False), (4096, 8190, True)])
def test_dequant_t_wide_tiles_bit_exact(device, K, N, with_zeros):
    """Shapes large enough for the 64-column tiles of cfa_w4a16_dequant_t (at
    least 1024 work-groups), with aligned 16-byte word loads and, at N = 8190,
    the one-word path; bit-exact against the [K, N] dequantisation."""
    g = torch.Generator().manual_seed(N)
    w = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    scales = (torch.rand(K // 128, N, generator=g) * 0.1 + 1e-3).half()
    zeros = torch.randint(0, 16, (K // 128, N), generator=g).half() if with_zeros else None
    q = pack_int4_weights(w).to(device)
    sd = scales.to(device)
    zd = zeros.to(device) if zeros is not None else None
    kn = w4a16_dequant(q, sd, zd, group_size=128)
    nk = w4a16_dequant(q, sd, zd, group_size=128, transposed=True)
    assert torch.equal(nk.view(torch.int16), kn.t().contiguous().view(torch.int16))


_ZP_SHAPES = [(504, 28672, 4096), (504, 6144, 4096), (504, 4096, 4096), (504, 4096, 14336),
              (1, 256, 128), (37, 256, 512), (600, 768, 1024), (8, 1024, 256), (16, 256, 8448),
              (300, 2304, 512)]


@pytest.mark.parametrize("M,N,K", _ZP_SHAPES)
@pytest.mark.parametrize("with_zeros", [True, False])
def test_gemm_zp_vs_dequantised_fp32(device, M, N, K, with_zeros):
    """cfa_w4a16_gemm_zp against an fp32 product of the bit-exact dequantised
    weights (the kernel dequantises exactly as cfa_w4a16_dequant): differences
    come from the fp32 accumulation order and the final bf16 rounding
    (tolerance 1e-2 of the output scale + 2^-7 relative).  The verify step's
    four target shapes (M = 504: QKV, O, gate/up, down), a single row, a
    partial row tile, three row tiles (M = 600), column tiles that are not a
    multiple of 8 (N = 768, 2304) and split-K shapes (the small ones leave
    CUs idle without a split; K = 8448 splits into odd slice counts)."""
    from cudaforge_amd.w4a16 import w4a16_gemm_zp

    g = torch.Generator().manual_seed(M + N + K + with_zeros)
    group = 128
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    w_int4 = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    scales = ((torch.rand(K // group, N, generator=g) * 0.5 + 0.5) / K ** 0.5).half().to(device)
    zeros = torch.full((K // group, N), 7.5, dtype=torch.float16, device=device) if with_zeros else None
    q = pack_int4_weights(w_int4).to(device)
    c = w4a16_gemm_zp(a, q, scales, zeros, group_size=group)
    w = w4a16_dequant(q, scales, zeros, group_size=group, dtype=torch.bfloat16).float()
    ref = a.float() @ w
    torch.cuda.synchronize()
    err = (c.float() - ref).abs()
    tol = 1e-2 * ref.abs().max() + 2.0 ** -7 * ref.abs()
    assert (err <= tol).all(), err.max().item()
    # reproducible: the same call gives the same bits
    c2 = w4a16_gemm_zp(a, q, scales, zeros, group_size=group)
    assert torch.equal(c, c2)


@pytest.mark.parametrize("M,N,K", [(504, 28672, 4096), (1, 512, 128), (37, 256, 512),
                                   (600, 768, 1024), (16, 512, 8448)])
def test_gemm_zp_silu_bit_exact(device, M, N, K):
    """cfa_w4a16_gemm_zp_silu equals cfa_w4a16_gemm_zp on the same
    interleaved gate/up weights, de-interleaved and passed through
    cfa_silu_mul, bit for bit: the target's gate/up shape (one K split), and
    split-K shapes whose partials the SiLU-gated reduce sums (M = 1, 16, 37)."""
    from cudaforge_amd.spec_step import deinterleave_gate_up, silu_mul
    from cudaforge_amd.w4a16 import w4a16_gemm_zp

    g = torch.Generator().manual_seed(7 * M + N + K)
    group = 128
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    q = pack_int4_weights(torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)).to(device)
    scales = ((torch.rand(K // group, N, generator=g) * 0.5 + 0.5) / K ** 0.5).half().to(device)
    zeros = torch.full((K // group, N), 7.5, dtype=torch.float16, device=device)
    fused = w4a16_gemm_zp(a, q, scales, zeros, group_size=group, silu=True)
    plain = silu_mul(deinterleave_gate_up(w4a16_gemm_zp(a, q, scales, zeros, group_size=group))
                     .contiguous())
    torch.cuda.synchronize()
    assert fused.shape == (M, N // 2)
    assert torch.equal(fused, plain)


@pytest.mark.parametrize("M,N,K", [(504, 4096, 4096), (504, 4096, 14336), (600, 768, 1024),
                                   (37, 256, 512), (16, 256, 768), (1, 256, 128)])
def test_gemm_zp_partials_rmsnorm_bit_exact(device, M, N, K):
    """The GEMM's split-K partials summed by cfa_rmsnorm_partials give the
    bits of cfa_w4a16_gemm_zp followed by cfa_rmsnorm (residual h and the
    normalised output), with 8, 4, 2, 3 (a count the kernel takes at run
    time) and 1 split(s) -- one split forced to fp32 partials as well."""
    from cudaforge_amd import _lib
    from cudaforge_amd.spec_step import add_norm_, rmsnorm_
    from cudaforge_amd.w4a16 import w4a16_gemm_zp, w4a16_gemm_zp_partials

    g = torch.Generator().manual_seed(3 * M + N + K)
    group = 128
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    q = pack_int4_weights(torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)).to(device)
    scales = ((torch.rand(K // group, N, generator=g) * 0.5 + 0.5) / K ** 0.5).half().to(device)
    zeros = torch.full((K // group, N), 7.5, dtype=torch.float16, device=device)
    h0 = torch.randn(M, N, generator=g).bfloat16().to(device)
    w = (1 + 0.1 * torch.randn(N, generator=g)).bfloat16().to(device)
    part = w4a16_gemm_zp_partials(a, q, scales, zeros, group_size=group)
    assert part.shape[0] == _lib.load().cfa_w4a16_gemm_zp_splits(M, N, K) >= 1
    h1, x1 = h0.clone(), torch.empty_like(h0)
    add_norm_(h1, part, w, 1e-5, x1)
    h2, x2 = h0.clone(), torch.empty_like(h0)
    rmsnorm_(h2, w4a16_gemm_zp(a, q, scales, zeros, group_size=group), w, 1e-5, x2)
    torch.cuda.synchronize()
    assert torch.equal(h1, h2) and torch.equal(x1, x2)


def test_gemm_zp_rejects_bad_shapes(device):
    from cudaforge_amd.w4a16 import w4a16_gemm_zp

    a = torch.randn(4, 128, device=device).bfloat16()
    q = torch.zeros(16, 100, dtype=torch.int32, device=device)  # N % 256 != 0
    s = torch.ones(1, 100, dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        w4a16_gemm_zp(a, q, s)
