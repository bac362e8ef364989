"""W4A16 weights in the reference's packed INT4 format.

``B_quant`` [K / 8, N] int32 holds nibble k % 8 of column n at bits
4 * (k % 8) of word (k // 8, n), unsigned 0..15, with fp16 group scales
[K / group, N] and optional fp16 zero points
(``csrc/include/cudaforge/kernels/dequantize.cuh:12-25``,
``tests/unit/test_int4_dequant.py:6-15``).  ``int4_gemm_dequant`` mirrors
``int4_gemm_dequant_triton`` (``csrc/kernels/triton/int4_dequant_triton.py:
86-131``): ``cfa_w4a16_dequant_t`` (the dequantised matrix written as
[N, K]) followed by a PyTorch-ROCm GEMM in the activations' dtype.  ``w4a16_gemm`` is the fused MFMA kernel
(``cfa_w4a16_gemm``: dequantisation in registers, no zero points).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from .verify import _stream_ptr

__all__ = ["pack_int4_weights", "w4a16_dequant", "w4a16_gemm", "w4a16_gemm_zp",
           "w4a16_gemm_zp_partials",
           "int4_gemm_dequant", "W4A16Linear"]


def pack_int4_weights(w_int4: torch.Tensor) -> torch.Tensor:
    """[K, N] values 0..15 -> [K // 8, N] int32, nibble k % 8 of word k // 8
    at bits 4 * (k % 8) (tests/unit/test_int4_dequant.py:6-15)."""
    K, N = w_int4.shape
    if K % 8:
        raise ValueError("K must be a multiple of 8")
    w = w_int4.to(torch.int32) & 0x0F
    packed = torch.zeros((K // 8, N), dtype=torch.int32, device=w.device)
    for i in range(8):
        packed |= w[i::8, :] << (i * 4)
    return packed


def w4a16_dequant(b_quant: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor] = None,
                  *, group_size: int = 128, dtype: torch.dtype = torch.bfloat16,
                  out: Optional[torch.Tensor] = None, transposed: bool = False) -> torch.Tensor:
    """Dequantise packed INT4 weights to [K, N] fp16 or bf16 on the device
    (cfa_w4a16_dequant); transposed=True writes the same values as [N, K]
    (cfa_w4a16_dequant_t), the layout the following GEMM runs fastest on."""
    if b_quant.dtype != torch.int32 or b_quant.device.type != "cuda" or b_quant.dim() != 2:
        raise ValueError("b_quant must be an int32 [K/8, N] HIP tensor")
    Kq, N = b_quant.shape
    K = Kq * 8
    if scales.dtype != torch.float16 or tuple(scales.shape) != (K // group_size, N):
        raise ValueError("scales must be fp16 [K/group_size, N]")
    if zeros is not None and (zeros.dtype != torch.float16 or zeros.shape != scales.shape):
        raise ValueError("zeros must be fp16 [K/group_size, N]")
    if dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("dtype must be float16 or bfloat16")
    shape = (N, K) if transposed else (K, N)
    if out is None:
        out = torch.empty(shape, dtype=dtype, device=b_quant.device)
    elif out.dtype != dtype or tuple(out.shape) != shape or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {list(shape)} tensor of `dtype`")
    bq, sc = b_quant.contiguous(), scales.contiguous()
    zz = zeros.contiguous() if zeros is not None else None
    fn = "cfa_w4a16_dequant_t" if transposed else "cfa_w4a16_dequant"
    with torch.cuda.device(b_quant.device):
        rc = getattr(_lib.load(), fn)(
            bq.data_ptr(), sc.data_ptr(), zz.data_ptr() if zz is not None else None, K, N,
            group_size, 1 if dtype == torch.bfloat16 else 0, out.data_ptr(),
            _stream_ptr(b_quant.device))
    _lib.check(rc, fn)
    return out


def fused_gemm_ok(a: torch.Tensor, b_quant: torch.Tensor, zeros, group_size: int) -> bool:
    """Whether cfa_w4a16_gemm takes this problem (else dequantise + GEMM)."""
    N = b_quant.shape[1]
    many_rows_bf16 = a.dtype == torch.bfloat16 and a.shape[0] > 64 and N % 64 == 0
    return (zeros is None and (N % 256 == 0 or many_rows_bf16) and group_size % 64 == 0
            and a.is_contiguous()
            and b_quant.is_contiguous() and a.data_ptr() % 16 == 0 and b_quant.data_ptr() % 16 == 0)


def w4a16_gemm(a: torch.Tensor, b_quant: torch.Tensor, scales: torch.Tensor, *,
               group_size: int = 128, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused a [M, K] (fp16 or bf16) x dequant(b_quant) -> [M, N] in a's dtype
    (cfa_w4a16_gemm)."""
    M, K = a.shape
    N = b_quant.shape[1]
    if b_quant.shape[0] * 8 != K:
        raise ValueError("K of a and b_quant differ")
    if out is None:
        out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    sc = scales.contiguous()
    with torch.cuda.device(a.device):
        rc = _lib.load().cfa_w4a16_gemm(a.data_ptr(), b_quant.data_ptr(), sc.data_ptr(), M, N, K,
                                        group_size, 1 if a.dtype == torch.float16 else 0,
                                        out.data_ptr(), _stream_ptr(a.device))
    _lib.check(rc, "cfa_w4a16_gemm")
    return out


def gemm_zp_ok(a: torch.Tensor, b_quant: torch.Tensor, group_size: int) -> bool:
    """Whether cfa_w4a16_gemm_zp takes this problem (else dequantise + GEMM)."""
    K, N = b_quant.shape[0] * 8, b_quant.shape[1]
    return (a.dtype == torch.bfloat16 and a.dim() == 2 and a.shape[1] == K and N % 256 == 0
            and K % 32 == 0 and group_size % 32 == 0 and K % group_size == 0
            and a.is_contiguous() and b_quant.is_contiguous() and a.data_ptr() % 16 == 0)


def w4a16_gemm_zp(a: torch.Tensor, b_quant: torch.Tensor, scales: torch.Tensor,
                  zeros: Optional[torch.Tensor] = None, *, group_size: int = 128,
                  out: Optional[torch.Tensor] = None,
                  workspace: Optional[torch.Tensor] = None, silu: bool = False) -> torch.Tensor:
    """Fused a [M, K] bf16 x W -> [M, N] bf16 with W = bf16((nibble - z) * s),
    the weights cfa_w4a16_dequant writes (cfa_w4a16_gemm_zp); `workspace`
    (uint8, cfa_w4a16_gemm_zp_workspace_size bytes) holds split-K partials.
    silu=True: W's columns are in the interleaved gate/up layout (64-column
    tile t = gate features 32t .. 32t + 31, then their up columns) and the
    result is silu(gate) * up, [M, N / 2] (cfa_w4a16_gemm_zp_silu),
    bit-identical to the plain product de-interleaved and passed through
    cfa_silu_mul."""
    if a.dtype != torch.bfloat16 or a.dim() != 2:
        raise ValueError("a must be a bf16 [M, K] tensor")
    M, K = a.shape
    N = b_quant.shape[1]
    if b_quant.shape[0] * 8 != K:
        raise ValueError("K of a and b_quant differ")
    if scales.dtype != torch.float16 or tuple(scales.shape) != (K // group_size, N):
        raise ValueError("scales must be fp16 [K/group_size, N]")
    if zeros is not None and (zeros.dtype != torch.float16 or zeros.shape != scales.shape):
        raise ValueError("zeros must be fp16 [K/group_size, N]")
    lib = _lib.load()
    need = lib.cfa_w4a16_gemm_zp_workspace_size(M, N, K)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=a.device)
    Nout = N // 2 if silu else N
    if out is None:
        out = torch.empty(M, Nout, dtype=torch.bfloat16, device=a.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (M, Nout) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bf16 [{M}, {Nout}] tensor")
    sc = scales.contiguous()
    zz = zeros.contiguous() if zeros is not None else None
    name = "cfa_w4a16_gemm_zp_silu" if silu else "cfa_w4a16_gemm_zp"
    with torch.cuda.device(a.device):
        rc = getattr(lib, name)(a.data_ptr(), b_quant.data_ptr(), sc.data_ptr(),
                                zz.data_ptr() if zz is not None else None, M, N, K,
                                group_size, out.data_ptr(), workspace.data_ptr(),
                                workspace.numel(), _stream_ptr(a.device))
    _lib.check(rc, name)
    return out


def w4a16_gemm_zp_partials(a: torch.Tensor, b_quant: torch.Tensor, scales: torch.Tensor,
                           zeros: Optional[torch.Tensor] = None, *, group_size: int = 128,
                           workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The fused product left as its split-K partials: fp32 [S, M, N]
    (cfa_w4a16_gemm_zp_partials), a view of `workspace` (uint8) when it is
    large enough; bf16 of their sum in slab order is w4a16_gemm_zp's result
    (cfa_rmsnorm_partials sums them)."""
    if a.dtype != torch.bfloat16 or a.dim() != 2:
        raise ValueError("a must be a bf16 [M, K] tensor")
    M, K = a.shape
    N = b_quant.shape[1]
    if b_quant.shape[0] * 8 != K:
        raise ValueError("K of a and b_quant differ")
    if scales.dtype != torch.float16 or tuple(scales.shape) != (K // group_size, N):
        raise ValueError("scales must be fp16 [K/group_size, N]")
    if zeros is not None and (zeros.dtype != torch.float16 or zeros.shape != scales.shape):
        raise ValueError("zeros must be fp16 [K/group_size, N]")
    lib = _lib.load()
    S = lib.cfa_w4a16_gemm_zp_splits(M, N, K)
    if S <= 0:
        raise ValueError("shape not taken by cfa_w4a16_gemm_zp (N % 256, K % 32)")
    need = S * M * N * 4
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        part = torch.empty(S, M, N, dtype=torch.float32, device=a.device)
    else:
        part = workspace.view(torch.uint8)[:need].view(torch.float32).view(S, M, N)
    sc = scales.contiguous()
    zz = zeros.contiguous() if zeros is not None else None
    with torch.cuda.device(a.device):
        rc = lib.cfa_w4a16_gemm_zp_partials(a.data_ptr(), b_quant.data_ptr(), sc.data_ptr(),
                                            zz.data_ptr() if zz is not None else None, M, N, K,
                                            group_size, part.data_ptr(), need,
                                            _stream_ptr(a.device))
    _lib.check(rc, "cfa_w4a16_gemm_zp_partials")
    return part


class W4A16Linear:
    """y = x @ W with W [K, N] held as packed INT4 + fp16 group scales and
    zero points, w = (nibble - z) * s (dequantize.cuh:12-25).
    Random initialisation: uniform nibbles, zero point 7.5 (symmetric
    weights), scales chosen so that the output of a unit-RMS input has RMS
    about 1.  With unsigned nibbles and no zero point every weight would be
    positive, and the residual stream of a random model grows to thousands
    and cancels on some rows, where no bf16 computation tracks an fp32 one."""

    def __init__(self, K: int, N: int, device, gen: torch.Generator, group: int = 128):
        self.K, self.N, self.group = K, N, group
        self.qweight = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), dtype=torch.int32,
                                     device=device, generator=gen)
        # E[(nibble - 7.5)^2] = 21.25 for uniform nibbles 0..15
        base = 1.0 / (math.sqrt(21.25) * math.sqrt(K))
        self.scales = (base * (0.5 + torch.rand(K // group, N, device=device, generator=gen))
                       ).to(torch.float16)
        self.zeros = torch.full_like(self.scales, 7.5)

    # class-wide switches: `fused_zp` (default) multiplies with
    # cfa_w4a16_gemm_zp, which dequantises in LDS per output tile, where the
    # shape allows (bf16, N % 256 == 0); at the verify step's M = 504 it takes
    # 51 / 42 / 150 / 85 us for QKV / O / gate-up / down against 51 / 43 / 175
    # / 110 us for dequantise + hipBLASLt.  `fused` selects the older
    # cfa_w4a16_gemm (no zero points) instead; off.
    fused_zp = True
    fused = False

    def __call__(self, x: torch.Tensor, scratch: torch.Tensor) -> torch.Tensor:
        if self.fused_zp and gemm_zp_ok(x, self.qweight, self.group):
            # the scratch that would hold the dequantised matrix holds the
            # split-K partials instead (at most 16 x M x N fp32, far less than
            # K x N bf16 at the model's shapes)
            ws = scratch.view(torch.uint8)
            return w4a16_gemm_zp(x, self.qweight, self.scales, self.zeros, group_size=self.group,
                                 workspace=ws)
        if self.fused and fused_gemm_ok(x, self.qweight, self.zeros, self.group):
            return w4a16_gemm(x, self.qweight, self.scales, group_size=self.group)
        # [N, K] (K contiguous): x @ w^T runs about 20% faster on hipBLASLt
        # than x @ w at M = 504 (1.27 against 1.06 PFLOP/s for gate/up)
        wt = scratch[: self.K * self.N].view(self.N, self.K)
        w4a16_dequant(self.qweight, self.scales, self.zeros, group_size=self.group,
                      dtype=x.dtype, out=wt, transposed=True)
        return x @ wt.t()

    def partials(self, x: torch.Tensor, scratch: torch.Tensor) -> torch.Tensor:
        """x @ W as fp32 split-K partials [S, M, N] in `scratch` (for a
        consumer that sums them, cfa_rmsnorm_partials) where the fused kernel
        takes the shape; else the bf16 product [M, N]."""
        if self.fused_zp and gemm_zp_ok(x, self.qweight, self.group):
            return w4a16_gemm_zp_partials(x, self.qweight, self.scales, self.zeros,
                                          group_size=self.group, workspace=scratch)
        return self(x, scratch)

    def silu_gated(self, x: torch.Tensor, scratch: torch.Tensor) -> torch.Tensor:
        """silu(x @ W_gate) * (x @ W_up) [M, N / 2] for W in the interleaved
        gate/up layout (64-column tile t = gate features 32t .. 32t + 31,
        then their up columns): the fused epilogue where cfa_w4a16_gemm_zp
        takes the shape, else the product de-interleaved and cfa_silu_mul."""
        if self.fused_zp and gemm_zp_ok(x, self.qweight, self.group):
            return w4a16_gemm_zp(x, self.qweight, self.scales, self.zeros, group_size=self.group,
                                 workspace=scratch.view(torch.uint8), silu=True)
        from .spec_step import deinterleave_gate_up, silu_mul
        return silu_mul(deinterleave_gate_up(self(x, scratch)).contiguous())


def int4_gemm_dequant(a: torch.Tensor, b_quant: torch.Tensor, scales: torch.Tensor,
                      zeros: Optional[torch.Tensor] = None, group_size: int = 128) -> torch.Tensor:
    """a [M, K] fp16 (or bf16) @ dequant(b_quant) -> [M, N] in a's dtype
    (fp32 accumulation), as int4_dequant_triton.py:86-131."""
    if a.dim() != 2 or a.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("a must be [M, K] fp16 or bf16")
    if b_quant.shape[0] * 8 != a.shape[1]:
        raise ValueError("K of a and b_quant differ")
    # dequantised as [N, K]: hipBLASLt multiplies a @ w^T about 20% faster
    # than a @ w at the verify step's shapes
    wt = w4a16_dequant(b_quant, scales, zeros, group_size=group_size, dtype=a.dtype,
                       transposed=True)
    return a @ wt.t()
