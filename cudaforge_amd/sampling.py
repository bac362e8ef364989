"""Token sampling on the GPU: plain decode and draft-tree expansion.

Mirrors the reference's two samplers:

* ``fused_sampling_triton(logits, temperature)``
  (``csrc/kernels/triton/sampling_triton.py:40-66``): the argmax of
  ``softmax(logits / T)``, i.e. of the logits, first index on ties;
* ``launch_fused_sampling`` / ``fused_sampling_kernel``
  (``csrc/include/cudaforge/engine/sampling.h:18-28, 61-216``): temperature
  <= 1e-5 is greedy (first argmax of the raw logits), otherwise one
  multinomial draw per row from ``softmax(logits / T)`` by the sequential fp32
  inverse CDF ``cdf += p_i; if (u <= cdf)``, V - 1 if none.  The reference
  kernel takes ``top_k`` / ``top_p`` but never applies them; so does this
  mirror.  Its uniforms come from cuRAND Philox seeded with ``rng_seed``; here
  they come from torch's generator seeded with ``rng_seed`` (another stream)
  or from the caller.

``sample`` is the general entry point (``cfa_sample``): multinomial,
filtered (top-p keep rule of ``cudaforge/speculative.py:67-81`` plus top-k,
renormalised), or greedy top-k; several independent draws per row.
``expand_tree_level`` uses it to draw the children of draft-tree nodes.

Every call runs on the HIP library; there is no CPU fallback.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .verify import _KINDS, _require_cuda, _stream_ptr

__all__ = [
    "SamplingParams",
    "sample",
    "sample_workspace_bytes",
    "fused_sampling_triton",
    "launch_fused_sampling",
    "expand_tree_level",
]

_SMODES = {"multinomial": _lib.CFA_SAMPLE_MULTINOMIAL, "filtered": _lib.CFA_SAMPLE_FILTERED,
           "greedy": _lib.CFA_SAMPLE_GREEDY}


@dataclass
class SamplingParams:
    """sampling.h:18-28 (device pointers become tensors)."""

    logits: Optional[torch.Tensor] = None         # [batch_size, vocab_size]
    output_tokens: Optional[torch.Tensor] = None  # [batch_size] int32
    batch_size: int = 0
    vocab_size: int = 0
    temperature: float = 1.0
    top_k: int = 50
    top_p: float = 0.9
    rng_seed: int = 1337


def sample_workspace_bytes(R: int, V: int, draws: int = 1, mode: str = "multinomial") -> int:
    return int(_lib.load().cfa_sample_workspace_size(R, V, draws, _SMODES[mode]))


def _rows_f32(x: torch.Tensor) -> torch.Tensor:
    if x.dtype in (torch.float16, torch.bfloat16):
        x = x.float()
    if x.dim() != 2:
        raise ValueError("rows must be [R, V]")
    if x.stride(1) != 1:
        x = x.contiguous()
    return x


def sample(rows: torch.Tensor, *, mode: str = "multinomial", temperature: float = 1.0,
           top_k: int = -1, top_p: float = 1.0, draws: int = 1,
           uniforms: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None,
           input_kind: str = "logits", return_probs: bool = False,
           workspace: Optional[torch.Tensor] = None):
    """Draw `draws` tokens from each of R rows ([R, V] logits or
    probabilities; fp32, or fp16/bf16 converted to fp32 first).

    mode "multinomial": softmax(row / T), sequential fp32 inverse CDF;
    "filtered": the top-p keep rule and top-k (<= 0: off), renormalised;
    "greedy": the `draws` largest values, largest first.  uniforms [R, draws]
    fp32 (drawn from `generator` when omitted: in (0, 1] for multinomial, in
    [0, 1) for filtered).  Returns int32
    [R, draws] (and the probabilities used, [R, V], with return_probs).
    """
    if mode not in _SMODES:
        raise ValueError(f"mode must be one of {sorted(_SMODES)}")
    if input_kind not in _KINDS:
        raise ValueError("input_kind must be 'logits' or 'probs'")
    if not isinstance(rows, torch.Tensor) or rows.device.type != "cuda":
        raise ValueError("rows must be a HIP device tensor")
    x = _rows_f32(rows)
    dev = x.device
    R, V = x.shape
    if draws < 1:
        raise ValueError("draws must be >= 1")
    out = torch.empty(R, draws, dtype=torch.int32, device=dev)
    probs = None
    u = None
    if mode != "greedy":
        if uniforms is None:
            u = torch.rand(R, draws, device=dev, generator=generator, dtype=torch.float32)
            if mode == "multinomial":
                # (0, 1], the range of curand_uniform: u = 0 would meet
                # `u <= cumulative` at index 0 whatever its probability
                # (the filtered draw takes the first prefix sum exceeding u
                # instead, so [0, 1) is right there)
                u = 1.0 - u
        else:
            _require_cuda("uniforms", uniforms, torch.float32, dev)
            if tuple(uniforms.shape) != (R, draws):
                raise ValueError("uniforms must be [R, draws]")
            u = uniforms.contiguous()
        if return_probs:
            probs = torch.empty(R, V, dtype=torch.float32, device=dev)
    elif return_probs:
        raise ValueError("greedy sampling produces no probabilities")
    need = sample_workspace_bytes(R, V, draws, mode)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().cfa_sample(
            x.data_ptr(), x.stride(0), _KINDS[input_kind], R, V, draws, float(temperature),
            int(top_k), float(top_p), _SMODES[mode], u.data_ptr() if u is not None else None,
            out.data_ptr(), probs.data_ptr() if probs is not None else None,
            workspace.data_ptr(), workspace.numel(), _stream_ptr(dev))
    _lib.check(rc, "cfa_sample")
    return (out, probs) if return_probs else out


def fused_sampling_triton(logits: torch.Tensor, temperature: float = 1.0) -> torch.Tensor:
    """sampling_triton.py:40-66: the argmax of softmax(logits / T) per row
    (the argmax of the logits; first index on ties).  int32 [batch_size]."""
    if logits.dim() != 2:
        raise ValueError("logits must be [batch_size, vocab_size]")
    return sample(logits, mode="greedy")[:, 0].contiguous()


def launch_fused_sampling(params: SamplingParams, stream: Optional[torch.cuda.Stream] = None,
                          uniforms: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sampling.h:195-216.  Writes params.output_tokens (allocated when None)
    and returns it."""
    x = params.logits
    if params.batch_size <= 0 or params.vocab_size <= 0 or x is None:
        raise ValueError("Invalid batch size or vocab size for sampling launch.")
    if x.dim() != 2 or tuple(x.shape) != (params.batch_size, params.vocab_size):
        raise ValueError("logits must be [batch_size, vocab_size]")
    ctx = torch.cuda.stream(stream) if stream is not None else _Null()
    with ctx:
        if params.temperature <= 1e-5:
            tok = sample(x, mode="greedy")[:, 0]
        else:
            gen = None
            if uniforms is None:
                gen = torch.Generator(device=x.device)
                gen.manual_seed(int(params.rng_seed))
            u = None if uniforms is None else uniforms.reshape(-1, 1).float()
            tok = sample(x, mode="multinomial", temperature=params.temperature, uniforms=u,
                         generator=gen)[:, 0]
        if params.output_tokens is None:
            params.output_tokens = torch.empty(params.batch_size, dtype=torch.int32,
                                               device=x.device)
        params.output_tokens.copy_(tok)
    return params.output_tokens


def expand_tree_level(draft_rows: torch.Tensor, *, children: int = 2, mode: str = "sample",
                      temperature: float = 1.0, uniforms: Optional[torch.Tensor] = None,
                      generator: Optional[torch.Generator] = None,
                      return_probs: bool = False):
    """Children of one level of draft-tree nodes: draft_rows [R, V] logits of
    the R nodes; returns int32 [R, children].

    mode "sample": i.i.d. draws from softmax(row / T) -- what multi-candidate
    rejection sampling (cfa_tree_verify, cpp mode) assumes of a node's
    children; "greedy": the `children` most likely tokens (greedy
    verification)."""
    if mode == "sample":
        return sample(draft_rows, mode="multinomial", temperature=temperature, draws=children,
                      uniforms=uniforms, generator=generator, return_probs=return_probs)
    if mode == "greedy":
        out = sample(draft_rows, mode="greedy", draws=children)
        return (out, None) if return_probs else out
    raise ValueError("mode must be 'sample' or 'greedy'")


class _Null:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False
