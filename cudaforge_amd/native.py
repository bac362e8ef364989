"""Compatibility layer for the reference's native speculative engine.

The reference exposes ``cudaforge.SpeculativeConfig``,
``cudaforge.SpeculativeVerificationResult`` and ``cudaforge.SpeculativeEngine``
from its pybind module (csrc/bindings/pybind_module.cpp:199-239, re-exported
at cudaforge/__init__.py:18-20), implemented by
csrc/include/cudaforge/scheduler/speculative.h:14-88 and
csrc/src/scheduler/speculative.cpp:8-150.  This module keeps those names, the
field names and defaults, the method names and keyword names, and the
uniform stream: the engine owns a ``std::mt19937`` seeded with ``rng_seed``
(held in libcfa.so, see cfa_rng_*) and consumes one draw per acceptance test
and one per final draw, as speculative.cpp:13-14, 64, 72 do.  The
verification itself runs on the GPU through ``cfa_chain_verify``.

Differences, all on inputs where the reference has undefined behaviour:
rows of different lengths, token ids outside [0, V), and (greedy) fewer than
K+1 target rows raise ``ValueError`` here.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .verify import chain_verify

_DIM_MSG = "Incompatible draft and target tensor dimensions in SpeculativeEngine."


@dataclass
class SpeculativeConfig:
    """speculative.h:14-19 (gamma, temperature and top_p are not read by verification)."""

    gamma: int = 5
    temperature: float = 1.0
    top_p: float = 1.0
    rng_seed: int = 42


@dataclass
class SpeculativeVerificationResult:
    """speculative.h:24-31."""

    accepted_tokens: List[int] = field(default_factory=list)
    final_token: int = 0
    num_accepted: int = 0
    end_of_sequence: bool = False


def _as_matrix(rows, name: str) -> np.ndarray:
    if isinstance(rows, torch.Tensor):
        a = rows.detach().to("cpu", torch.float32).numpy()
    elif isinstance(rows, np.ndarray):
        a = rows.astype(np.float32, copy=False)
    else:
        rows = list(rows)
        lens = {len(r) for r in rows}
        if len(lens) > 1:
            raise ValueError(f"{name}: every row must have the same vocabulary size")
        a = np.asarray(rows, dtype=np.float32)
    if a.ndim == 1 and a.size == 0:
        a = a.reshape(0, 0)
    if a.ndim != 2:
        raise ValueError(f"{name} must be a list of rows")
    return np.ascontiguousarray(a)


class SpeculativeEngine:
    """Per-sequence verification with the reference's RNG stream (speculative.h:37-88)."""

    def __init__(self, config: SpeculativeConfig, device: Optional[torch.device] = None) -> None:
        self._config = SpeculativeConfig(**vars(config))
        self._device = torch.device(device) if device is not None else torch.device("cuda", 0)
        lib = _lib.load()
        self._rng = lib.cfa_rng_create(ctypes.c_uint64(int(config.rng_seed) & (2**64 - 1)))
        if not self._rng:
            raise RuntimeError("cfa_rng_create failed")

    def __del__(self) -> None:
        rng = getattr(self, "_rng", None)
        if rng:
            _lib.load().cfa_rng_destroy(rng)
            self._rng = None

    # set_config does not reseed the stream (speculative.h:70-73).
    def set_config(self, config: SpeculativeConfig) -> None:
        self._config = SpeculativeConfig(**vars(config))

    def get_config(self) -> SpeculativeConfig:
        return SpeculativeConfig(**vars(self._config))

    def _peek(self, n: int) -> np.ndarray:
        out = np.zeros(max(n, 1), np.float32)
        _lib.check(_lib.load().cfa_rng_peek(self._rng, n, out.ctypes.data_as(_lib._f32p)),
                   "cfa_rng_peek")
        return out[:n]

    def _advance(self, n: int) -> None:
        _lib.check(_lib.load().cfa_rng_advance(self._rng, n), "cfa_rng_advance")

    def _run(self, draft_tokens: Sequence[int], draft_probs, target_probs, eos_token_id: int,
             greedy: bool) -> SpeculativeVerificationResult:
        toks = np.asarray(list(draft_tokens), dtype=np.int64).reshape(-1)
        K = toks.size
        t = _as_matrix(target_probs, "target_probs")
        if greedy:
            if t.shape[0] < K + 1:
                raise ValueError(_DIM_MSG)
            d = np.zeros((0, t.shape[1]), np.float32)
        else:
            d = _as_matrix(draft_probs, "draft_probs") if K or len(draft_probs) else \
                np.zeros((0, t.shape[1]), np.float32)
            if d.shape[0] != K or t.shape[0] < K + 1:  # speculative.cpp:58-62
                raise ValueError(_DIM_MSG)
            if K and d.shape[1] != t.shape[1]:
                raise ValueError("draft_probs and target_probs must share the vocabulary size")
        V = t.shape[1]
        if V <= 0:
            raise ValueError("vocabulary size must be positive")
        if K and (toks.min() < 0 or toks.max() >= V):
            raise ValueError("draft token id outside [0, vocab_size)")
        dev = self._device
        tt = torch.from_numpy(t[: K + 1]).to(dev).unsqueeze(0)
        tk = torch.from_numpy(toks.astype(np.int32)).to(dev).unsqueeze(0)
        if greedy:
            out = chain_verify(tt, None, tk, None, input_kind="probs", mode="greedy",
                               eos_token_id=eos_token_id)
        else:
            U = self._peek(K + 1)
            dd = torch.from_numpy(d).to(dev).unsqueeze(0)
            uu = torch.from_numpy(U).to(dev).unsqueeze(0)
            out = chain_verify(tt, dd, tk, uu, input_kind="probs", mode="cpp",
                               eos_token_id=eos_token_id)
        n = int(out.accept_len[0].item())
        fin = int(out.final[0].item())
        eos = bool(out.eos[0].item())
        accepted = [int(x) for x in toks[:n]]
        if not greedy:
            eos_accepted = n > 0 and accepted[-1] == eos_token_id
            # one draw per test, plus the final draw unless an EOS was accepted
            draws = n if eos_accepted else (n + 2 if n < K else K + 1)
            self._advance(draws)
        return SpeculativeVerificationResult(accepted_tokens=accepted, final_token=fin,
                                             num_accepted=n, end_of_sequence=eos)

    def verify_candidates(self, draft_tokens, draft_probs, target_probs,
                          eos_token_id: int) -> SpeculativeVerificationResult:
        """speculative.cpp:50-103."""
        return self._run(draft_tokens, draft_probs, target_probs, eos_token_id, greedy=False)

    def verify_candidates_greedy(self, draft_tokens, target_probs,
                                 eos_token_id: int) -> SpeculativeVerificationResult:
        """speculative.cpp:105-150."""
        return self._run(draft_tokens, None, target_probs, eos_token_id, greedy=True)
