"""Drop-in replacement for ``cudaforge/speculative.py`` (Bahaa-Labs/CUDAForge).

Same public names, signatures, defaults and result fields as the reference:

  SpeculativeBatchResult           cudaforge/speculative.py:15-24
  SpeculativeEngine.__init__       cudaforge/speculative.py:30-55
  SpeculativeEngine._sample_next_token   :57-84
  SpeculativeEngine.step           cudaforge/speculative.py:86-211
  SpeculativeEngine.get_aggregate_acceptance_rate   :213-217

What changes is the verification phase: the reference stacks draft
probabilities, softmaxes the target window and loops over positions with a
device-to-host sync per position (speculative.py:118-185).  Here the target
logits window and the stacked draft logits go straight to the fused HIP
kernel (softmax + acceptance + resample/bonus in one pass over the logits) and
the host synchronises once, to learn the accept length.

Randomness.  The reference draws acceptance uniforms with ``torch.rand_like``
(:161) and resamples with ``torch.multinomial`` (:182, :84).  Here one
``torch.rand([B, K+2])`` supplies all of them: columns 0..K-1 are the
acceptance draws, column K drives an inverse-CDF draw for the resample /
bonus token and column K+1 the bonus that follows a rejection at the last
position.  Acceptance decisions therefore follow the reference rule exactly
for the same uniforms; resampled and bonus ids follow the same distributions
as ``torch.multinomial`` but are not the same ids for a seed.  An optional
``generator`` (keyword-only, default: torch's global generator, as the
reference) drives the draft draws and these uniforms; the uniforms of each
step are returned in ``SpeculativeBatchResult.uniforms``.

Reference behaviour kept: ``num_accepted`` counts the resampled or bonus token
(:184, :195) and ``acceptance_rate = num_accepted / K`` can exceed 1; a
rejection at the last draft position (i = K-1) brings num_accepted to K, so
the ``num_accepted == self.k`` branch (:188) appends a bonus token as well
(K+1 tokens, rate (K+1)/K).  K = 0 fails where the reference fails: the
``torch.cat`` of the empty draft list (:128) raises ``ValueError`` before the
target runs, and the lifetime totals are left unchanged.  An empty batch
accepts all K drafts and the bonus, as the reference's ``.all()`` over no
rows does (:166): ``accepted_tokens`` is [0, K+1].

``verify_mode="python"`` (default) keeps the reference's batch lock-step rule
(one accept count n for the whole batch, :166).  ``verify_mode="cpp"`` applies
the per-sequence rule of ``csrc/src/scheduler/speculative.cpp:50-103`` instead;
rows then accept different counts, ``accepted_tokens`` is padded with -1 and
``num_accepted`` is the widest row's count.
"""
from __future__ import annotations

import dataclasses
import time
from typing import Any, Dict, List, Optional

import torch
import torch.nn.functional as F

from .verify import chain_verify


@dataclasses.dataclass
class SpeculativeBatchResult:
    """Holds execution result metrics for a speculative step (speculative.py:15-24)."""

    accepted_tokens: torch.Tensor  # [batch_size, num_accepted]
    num_accepted: int
    draft_tokens_generated: int
    acceptance_rate: float
    draft_latency_ms: float
    target_latency_ms: float
    # per-row emitted counts ("cpp" verify mode; None in the reference's mode)
    num_emitted_per_row: Optional[torch.Tensor] = None
    # the step's uniforms [B, K+2] (python mode) / [B, K+1] (cpp mode)
    uniforms: Optional[torch.Tensor] = None


def _sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


class SpeculativeEngine:
    """Speculative decoding engine whose verification runs on gfx950 HIP kernels."""

    def __init__(
        self,
        draft_runner: Any,
        target_runner: Any,
        num_speculative_tokens: int = 5,
        temperature: float = 1.0,
        top_p: float = 0.9,
        verify_mode: str = "python",
        *,
        generator: Optional[torch.Generator] = None,
    ) -> None:
        if verify_mode not in ("python", "cpp"):
            raise ValueError("verify_mode must be 'python' or 'cpp'")
        self.draft_runner = draft_runner
        self.target_runner = target_runner
        self.k = num_speculative_tokens
        self.temperature = max(temperature, 1e-5)  # speculative.py:50
        self.top_p = top_p
        self.verify_mode = verify_mode
        self.generator = generator

        self.total_draft_tokens: int = 0
        self.total_accepted_tokens: int = 0

    def _rand(self, *shape: int, device: torch.device) -> torch.Tensor:
        return torch.rand(*shape, device=device, dtype=torch.float32, generator=self.generator)

    def _draw_draft(self, probs: torch.Tensor) -> torch.Tensor:
        """One draft token per row from the draft softmax (speculative.py:119)."""
        return torch.multinomial(probs, num_samples=1, generator=self.generator)

    @torch.no_grad()
    def _sample_next_token(
        self,
        logits: torch.Tensor,
        temperature: float = 1.0,
        top_p: float = 0.9,
    ) -> torch.Tensor:
        """Temperature, top-p filter and one draw per row (speculative.py:57-84).

        logits [B, V] on a HIP device; returns [B, 1] int64.  Runs the fused
        kernel with K = 0 draft tokens: only its python-mode bonus draw remains.
        """
        if logits.dim() != 2:
            raise ValueError("logits must be [B, V]")
        B = logits.shape[0]
        if B == 0:
            return torch.empty(0, 1, dtype=torch.long, device=logits.device)
        x = logits.float().contiguous().unsqueeze(1)
        u = self._rand(B, 2, device=logits.device)
        tok = torch.empty(B, 0, dtype=torch.int32, device=logits.device)
        out = chain_verify(x, x[:, :0], tok, u, input_kind="logits",
                           temperature=temperature, top_p=top_p, mode="python")
        return out.final.long().unsqueeze(1)

    @torch.no_grad()
    def step(
        self,
        input_ids: torch.Tensor,
        kv_cache_handles: Optional[Dict[str, Any]] = None,
    ) -> SpeculativeBatchResult:
        """One round of drafting, target verification and rejection sampling."""
        device = input_ids.device
        batch_size = input_ids.shape[0]
        K = self.k

        # Phase 1: draft proposals (speculative.py:107-131).  The draft's logits
        # are kept; their softmax is recomputed inside the verification kernel.
        t0 = time.perf_counter()
        draft_input_ids = input_ids.clone()
        draft_tokens_list: List[torch.Tensor] = []
        draft_logits_list: List[torch.Tensor] = []
        for _ in range(K):
            draft_logits = self.draft_runner.forward(draft_input_ids, kv_cache_handles)
            next_logits = draft_logits[:, -1, :].float()
            probs = F.softmax(next_logits / self.temperature, dim=-1)
            next_token = self._draw_draft(probs)
            draft_tokens_list.append(next_token)
            draft_logits_list.append(next_logits)
            draft_input_ids = torch.cat([draft_input_ids, next_token], dim=-1)
        _sync(device)
        t_draft_ms = (time.perf_counter() - t0) * 1000.0

        # With K = 0 this raises ValueError, as speculative.py:128 does.
        draft_tokens = torch.cat(draft_tokens_list, dim=-1)
        draft_logits = torch.stack(draft_logits_list, dim=1)  # [B, K, V]

        # Phase 2: target forward (speculative.py:136-147).
        t1 = time.perf_counter()
        verification_input_ids = torch.cat([input_ids, draft_tokens], dim=-1)
        target_logits = self.target_runner.forward(verification_input_ids, kv_cache_handles)
        window = target_logits[:, -(K + 1):, :]
        if window.dtype != torch.float32:
            window = window.float()
        _sync(device)
        t_target_ms = (time.perf_counter() - t1) * 1000.0

        # Phase 3: fused softmax + rejection sampling + resample/bonus.
        python = self.verify_mode == "python"
        uniforms = self._rand(batch_size, K + (2 if python else 1), device=device)
        if batch_size == 0:
            # No row rejects: python mode accepts all K drafts and appends the
            # bonus (speculative.py:166, :188); a cpp-mode row emits at least
            # its final token.
            width = K + 1 if python else 1
            accepted_tokens = torch.empty(0, width, dtype=torch.long, device=device)
            per_row = None if python else torch.empty(0, dtype=torch.int32, device=device)
        else:
            res = chain_verify(
                window, draft_logits, draft_tokens.to(torch.int32), uniforms,
                input_kind="logits", temperature=self.temperature, top_p=self.top_p,
                mode=self.verify_mode)
            # one host sync: the emitted count (equal on every row in python mode)
            width = int(res.num_emitted.max().item())
            accepted_tokens = res.tokens[:, :width].long()
            per_row = None if python else res.num_emitted
        num_accepted = width
        self.total_draft_tokens += K
        self.total_accepted_tokens += num_accepted
        acceptance_rate = num_accepted / K

        return SpeculativeBatchResult(
            accepted_tokens=accepted_tokens,
            num_accepted=num_accepted,
            draft_tokens_generated=K,
            acceptance_rate=acceptance_rate,
            draft_latency_ms=t_draft_ms,
            target_latency_ms=t_target_ms,
            num_emitted_per_row=per_row,
            uniforms=uniforms,
        )

    def get_aggregate_acceptance_rate(self) -> float:
        """Overall accepted / drafted ratio (speculative.py:213-217)."""
        if self.total_draft_tokens == 0:
            return 0.0
        return self.total_accepted_tokens / self.total_draft_tokens
