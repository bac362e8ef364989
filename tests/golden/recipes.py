"""Seeded input recipes shared by the golden-vector writer and the tests.

Only numpy's ``default_rng`` (PCG64) ``standard_normal`` / ``random`` streams
are used; the large-V fixtures store a SHA-256 of the generated inputs so a
change of stream is detected rather than silently compared.
"""
from __future__ import annotations

import numpy as np


def _softmax64(x: np.ndarray) -> np.ndarray:
    x = x - x.max(axis=-1, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=-1, keepdims=True)


def _draw(p: np.ndarray, u: float) -> int:
    c = np.cumsum(p)
    return int(min(np.searchsorted(c, u * c[-1], side="right"), p.size - 1))


def chain_case(seed: int, calls: int, K: int, V: int, sigma: float = 2.0, onehot: bool = False,
               eos_bias: bool = False, equal: bool = False, zero_q: bool = False):
    """Inputs for `calls` successive chain verifications of K drafts over V.

    Returns tokens [C,K] int32, dprobs [C,K,V] fp32, tprobs [C,K+1,V] fp32, eos.
    target logits ~ sigma * N(0,1); draft logits = target + 0.5 * N(0,1);
    drafts are drawn from the draft distribution.
      onehot   : one-hot rows (greedy-style known answers)
      eos_bias : token 0 is EOS and is favoured (+3 logits) so it is drawn often
      equal    : draft row = target row except a doubled draft probability at
                 the drafted token (residual sum 0 -> target fallback)
      zero_q   : the draft probability of some drafted tokens is 0
    """
    rng = np.random.default_rng(seed)
    C = calls
    tl = sigma * rng.standard_normal((C, K + 1, V))
    dl = tl[:, :K] + 0.5 * rng.standard_normal((C, K, V))
    eos = -1
    if eos_bias:
        eos = 0
        tl[..., 0] += 3.0
        dl[..., 0] += 3.0
    if onehot:
        tp = np.zeros((C, K + 1, V))
        dp = np.zeros((C, K, V))
        hot_t = rng.integers(0, V, (C, K + 1))
        hot_d = np.where(rng.random((C, K)) < 0.7, hot_t[:, :K], rng.integers(0, V, (C, K)))
        for c in range(C):
            for i in range(K + 1):
                tp[c, i, hot_t[c, i]] = 1.0
            for i in range(K):
                dp[c, i, hot_d[c, i]] = 1.0
    else:
        tp = _softmax64(tl)
        dp = _softmax64(dl)
    u = rng.random((C, K))
    tok = np.zeros((C, K), np.int32)
    for c in range(C):
        for i in range(K):
            tok[c, i] = _draw(dp[c, i], u[c, i])
    if equal:
        dp = tp[:, :K].copy()
        for c in range(C):
            for i in range(K):
                dp[c, i, tok[c, i]] *= 2.0
    if zero_q:
        z = rng.random((C, K)) < 0.5
        for c in range(C):
            for i in range(K):
                if z[c, i]:
                    dp[c, i, tok[c, i]] = 0.0
    return tok, dp.astype(np.float32), tp.astype(np.float32), eos


def c2_inputs(seed: int, B: int = 64, K: int = 8, V: int = 128256, sigma: float = 2.0,
              noise: float = 0.5, temperature: float = 0.7):
    """The chain-sampling benchmark workload (B=64, K=8, V=128256) as numpy:
    target logits [B,K+1,V] = sigma * N(0,1); draft logits [B,K,V] = target
    + noise * N(0,1); drafts drawn from softmax(draft / T); uniforms [B,K+1]."""
    rng = np.random.default_rng(seed)
    tl = (sigma * rng.standard_normal((B, K + 1, V))).astype(np.float32)
    dl = (tl[:, :K] + noise * rng.standard_normal((B, K, V))).astype(np.float32)
    dp = _softmax64(dl.astype(np.float64) / temperature)
    u = rng.random((B, K))
    tok = np.zeros((B, K), np.int32)
    for b in range(B):
        for i in range(K):
            tok[b, i] = _draw(dp[b, i], u[b, i])
    U = rng.random((B, K + 1)).astype(np.float32)
    return tl, dl, tok, U
