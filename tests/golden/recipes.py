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


# ---- python-engine step cases (cudaforge/speculative.py:86-211) ----------

def python_step_case(seed: int, B: int, K: int, V: int, steps: int, sigma: float = 2.0,
                     noise: float = 0.5):
    """Logit tables and uniforms for `steps` successive steps of the python engine.

    Returns draft [S,B,K,V] fp32 (the last-row logits of each of the K draft
    forwards), target [S,B,K+1,V] fp32 (the target's last K+1 rows) and
    uniforms: draft draws [S,B,K], acceptance draws [S,B,K], final draws
    [S,B,2] (the resample or bonus, then the bonus after a rejection at the
    last position), all fp32 in [0, 1).  target = sigma * N(0,1);
    draft = target[:K] + noise * N(0,1)."""
    rng = np.random.default_rng(seed)
    tl = (sigma * rng.standard_normal((steps, B, K + 1, V))).astype(np.float32)
    dl = (tl[:, :, :K] + noise * rng.standard_normal((steps, B, K, V))).astype(np.float32)
    ud = rng.random((steps, B, K)).astype(np.float32)
    ua = rng.random((steps, B, K)).astype(np.float32)
    uf = rng.random((steps, B, 2)).astype(np.float32)
    return dl, tl, ud, ua, uf


def fed_inverse_cdf(w: np.ndarray, u: np.ndarray):
    """Stand-in for torch.multinomial(w, 1) driven by fed uniforms: per row, the
    first index whose fp64 prefix sum of w / sum(w) exceeds u (a zero-weight
    index is never returned).  Also returns each draw's distance from u to the
    nearest prefix-sum boundary of its interval, so that a comparison with a
    draw computed in another precision can leave out draws within rounding of
    a boundary."""
    w = np.asarray(w, np.float64)
    ids = np.zeros(w.shape[0], np.int64)
    margin = np.zeros(w.shape[0], np.float64)
    for r in range(w.shape[0]):
        c = np.cumsum(w[r] / w[r].sum())
        i = int(np.searchsorted(c, float(u[r]), side="right"))
        if i >= c.size:  # u past the last prefix sum: the last positive weight
            i = int(np.flatnonzero(w[r] > 0)[-1])
        lo = c[i - 1] if i > 0 else 0.0
        ids[r] = i
        margin[r] = min(abs(float(u[r]) - lo), abs(c[i] - float(u[r])))
    return ids, margin


class TableRunner:
    """A runner with the protocol of speculative.py:115,139 (``forward(input_ids,
    kv_cache_handles) -> logits [B, T, V]``) that replays logit tables.

    table [S, B, R, V].  As the draft runner (``per_step`` = K forwards per
    step), forward call j of step s returns logits whose last row is
    table[s, :, j]; as the target runner (one forward per step) the last R
    rows are table[s].  Other rows are zero: the engine never reads them."""

    def __init__(self, table, draft: bool, device="cpu"):
        import torch

        self.table = torch.as_tensor(np.ascontiguousarray(table)).to(device)
        self.draft = draft
        self.calls = 0
        self.inputs = []

    def forward(self, input_ids, kv_cache_handles=None):
        import torch

        S, B, R, V = self.table.shape
        self.inputs.append(input_ids.detach().cpu().clone())
        T = input_ids.shape[1]
        out = torch.zeros(input_ids.shape[0], T, V, dtype=self.table.dtype,
                          device=self.table.device)
        if self.draft:
            s, j = divmod(self.calls, R)
            out[:, -1] = self.table[s, :, j]
        else:
            out[:, T - R:] = self.table[self.calls]
        self.calls += 1
        return out
