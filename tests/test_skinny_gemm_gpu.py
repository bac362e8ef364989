"""GPU tier: cfa_gemm_bf16_skinny (few-row bf16 GEMM) against a float64
product of the same bf16 operands.  Tolerance: one bf16 rounding of the
output (2^-8 relative) plus 2^-14 of |a| @ |w| for the fp32 accumulation
order."""
import pytest
import torch

from cudaforge_amd.spec_step import (deinterleave_gate_up, interleave_gate_up, silu_mul,
                                     skinny_gemm, skinny_gemm_silu, skinny_gemm_workspace_bytes)

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed=0):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(K, N, generator=g) / K ** 0.5).bfloat16()
    return a, w


def _check(out, a, w):
    ref = a.double() @ w.double()
    bound = ref.abs() * 2.0 ** -8 + (a.double().abs() @ w.double().abs()) * 2.0 ** -14
    err = (out.double().cpu() - ref).abs()
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}"


def _workspace(device, M, N, K, splits):
    n = skinny_gemm_workspace_bytes(M, N, K, splits)
    return torch.zeros(max(n, 65536), dtype=torch.uint8, device=device)


@pytest.mark.parametrize("M", [1, 8, 16, 17, 32, 33, 64, 65, 100, 128])
@pytest.mark.parametrize("splits", [1, 2, 0])
def test_small_shapes(device, M, splits):
    N, K = 192, 512
    a, w = _operands(M, N, K, seed=M)
    ws = _workspace(device, M, N, K, splits)
    out = skinny_gemm(a.to(device), w.to(device), ws, splits=splits)
    torch.cuda.synchronize()
    _check(out, a, w)
    # the arrival counters are left at zero
    assert int(ws[:65536].count_nonzero()) == 0


@pytest.mark.parametrize("M,N,K", [(8, 3072, 2048), (64, 2048, 2048), (128, 16384, 2048),
                                   (16, 2048, 8192), (128, 2048, 8192)])
def test_draft_shapes(device, M, N, K):
    """The draft model's projections (QKV, O, gate/up, down) at level sizes,
    with the library's split choice; bitwise equal on a repeat."""
    a, w = _operands(M, N, K, seed=N + M)
    ad, wd = a.to(device), w.to(device)
    ws = _workspace(device, M, N, K, 0)
    out1 = skinny_gemm(ad, wd, ws)
    out2 = skinny_gemm(ad, wd, ws)
    torch.cuda.synchronize()
    _check(out1, a, w)
    assert torch.equal(out1, out2)


def test_split_counts_agree(device):
    """Every split count gives a correct result (partials summed in split
    order), one workspace shared by calls of different shapes."""
    M, N, K = 40, 4096, 2048
    a, w = _operands(M, N, K, seed=5)
    ad, wd = a.to(device), w.to(device)
    ws2 = w[:, :128].contiguous()
    ws = _workspace(device, M, N, K, 16)
    for S in (1, 2, 4, 8, 16):
        out = skinny_gemm(ad, wd, ws, splits=S)
        small = skinny_gemm(ad[:3], ws2.to(device), ws, splits=S)
        torch.cuda.synchronize()
        _check(out, a, w)
        _check(small, a[:3], ws2)
    assert int(ws[:65536].count_nonzero()) == 0


def test_rejects_bad_operands(device):
    a = torch.zeros(8, 256, dtype=torch.float32, device=device)
    w = torch.zeros(256, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        skinny_gemm(a, w)
    with pytest.raises(ValueError):
        skinny_gemm(a.bfloat16(), w.t().contiguous().t())


def test_gate_up_layout_round_trip():
    w = torch.arange(3 * 256, dtype=torch.float32).view(3, 256)
    il = interleave_gate_up(w)
    assert torch.equal(il[:, :32], w[:, :32]) and torch.equal(il[:, 32:64], w[:, 128:160])
    assert torch.equal(deinterleave_gate_up(il), w)


@pytest.mark.parametrize("M", [1, 8, 17, 64, 128])
@pytest.mark.parametrize("splits", [1, 2, 0])
def test_silu_epilogue_bit_exact(device, M, splits):
    """cfa_gemm_bf16_skinny_silu equals the plain product on the same
    interleaved weights, de-interleaved, followed by cfa_silu_mul -- bit for
    bit (the same sums, the same roundings)."""
    K, F = 512, 384
    g = torch.Generator().manual_seed(100 + M)
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    w = (torch.randn(K, 2 * F, generator=g) * 2 / K ** 0.5).bfloat16()
    w_il = interleave_gate_up(w).to(device)
    ws = _workspace(device, M, 2 * F, K, splits)
    fused = skinny_gemm_silu(a, w_il, ws, splits=splits)
    plain = silu_mul(deinterleave_gate_up(skinny_gemm(a, w_il, ws, splits=splits)).contiguous())
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))
    assert int(ws[:65536].count_nonzero()) == 0
