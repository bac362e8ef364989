"""Random-init model runners for the chain speculative step.

``cudaforge/speculative.py`` drives two duck-typed runners through one call,
``runner.forward(input_ids, kv_cache_handles) -> logits [B, T, V]``
(speculative.py:115, :139-141); the reference ships no runner of its own.
``DecoderRunner`` is a small pre-norm causal decoder (RMSNorm, multi-head
attention with rotary positions, SiLU-gated MLP, untied LM head) with seeded
random weights, so a CPU copy and a HIP copy built from the same seed hold
identical weights.  Like the reference's call pattern it recomputes the whole
prefix on every call (no KV cache); ``kv_cache_handles`` is accepted and
ignored.

The two shapes of the reference's CPU speculative step are provided:
``target_runner()`` (4 layers, d 512, 8 heads of 64) and ``draft_runner()``
(1 layer, d 256, 4 heads of 64), both over a 32000-token vocabulary.
"""
from __future__ import annotations

import math
from typing import Any, Optional

import torch
import torch.nn.functional as F


class DecoderRunner:
    """Pre-norm causal decoder with seeded random weights (fp32 by default)."""

    def __init__(self, vocab: int, d_model: int, n_layers: int, n_heads: int,
                 head_dim: int = 64, ffn: Optional[int] = None, seed: int = 0,
                 device: Any = "cpu", dtype: torch.dtype = torch.float32,
                 rope_theta: float = 10000.0, init_std: float = 0.02) -> None:
        self.vocab, self.d, self.L = vocab, d_model, n_layers
        self.H, self.Dh = n_heads, head_dim
        self.F = ffn or 4 * d_model
        self.theta = rope_theta
        self.device = torch.device(device)
        self.dtype = dtype
        g = torch.Generator().manual_seed(seed)

        def w(*shape, std=init_std):
            return (torch.randn(*shape, generator=g) * std).to(self.device, dtype)

        hd = n_heads * head_dim
        self.embed = w(vocab, d_model, std=1.0)
        self.layers = []
        for _ in range(n_layers):
            self.layers.append(dict(
                n1=torch.ones(d_model, device=self.device, dtype=dtype),
                wqkv=w(d_model, 3 * hd), wo=w(hd, d_model),
                n2=torch.ones(d_model, device=self.device, dtype=dtype),
                wgu=w(d_model, 2 * self.F), wd=w(self.F, d_model)))
        self.norm = torch.ones(d_model, device=self.device, dtype=dtype)
        self.head = w(d_model, vocab, std=1.0 / math.sqrt(d_model))

    def to(self, device: Any) -> "DecoderRunner":
        """A copy of this runner on `device` (same weights)."""
        out = object.__new__(DecoderRunner)
        out.__dict__.update(self.__dict__)
        out.device = torch.device(device)
        out.embed = self.embed.to(device)
        out.layers = [{k: v.to(device) for k, v in lay.items()} for lay in self.layers]
        out.norm = self.norm.to(device)
        out.head = self.head.to(device)
        return out

    @staticmethod
    def _rms(x: torch.Tensor, wgt: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * wgt

    def _rope(self, x: torch.Tensor) -> torch.Tensor:
        # x [B, H, T, Dh]: rotate-half rotary embedding at positions 0..T-1
        T, Dh = x.shape[-2], x.shape[-1]
        inv = self.theta ** (-torch.arange(0, Dh, 2, device=x.device, dtype=torch.float32) / Dh)
        ang = torch.arange(T, device=x.device, dtype=torch.float32)[:, None] * inv[None, :]
        cos = torch.cat([ang.cos(), ang.cos()], -1).to(x.dtype)
        sin = torch.cat([ang.sin(), ang.sin()], -1).to(x.dtype)
        x1, x2 = x[..., : Dh // 2], x[..., Dh // 2:]
        return x * cos + torch.cat([-x2, x1], -1) * sin

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, kv_cache_handles: Any = None) -> torch.Tensor:
        """input_ids [B, T] int64 -> logits [B, T, vocab] (the runner protocol of
        speculative.py:115, :139-141)."""
        B, T = input_ids.shape
        h = self.embed[input_ids]
        for lay in self.layers:
            x = self._rms(h, lay["n1"])
            qkv = (x @ lay["wqkv"]).view(B, T, 3, self.H, self.Dh).permute(2, 0, 3, 1, 4)
            q, k, v = self._rope(qkv[0]), self._rope(qkv[1]), qkv[2].contiguous()
            a = F.scaled_dot_product_attention(q.contiguous(), k.contiguous(), v, is_causal=True)
            h = h + a.transpose(1, 2).reshape(B, T, self.H * self.Dh) @ lay["wo"]
            x = self._rms(h, lay["n2"])
            gu = x @ lay["wgu"]
            h = h + (F.silu(gu[..., : self.F]) * gu[..., self.F:]) @ lay["wd"]
        return self._rms(h, self.norm) @ self.head


def target_runner(seed: int = 1, device: Any = "cpu", vocab: int = 32000) -> DecoderRunner:
    """4 layers, d_model 512, 8 heads of 64, fp32."""
    return DecoderRunner(vocab, 512, 4, 8, 64, seed=seed, device=device)


def draft_runner(seed: int = 2, device: Any = "cpu", vocab: int = 32000) -> DecoderRunner:
    """1 layer, d_model 256, 4 heads of 64, fp32."""
    return DecoderRunner(vocab, 256, 1, 4, 64, seed=seed, device=device)
