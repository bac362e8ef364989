"""CPU tier: the python-mode oracle (oracle.python_verify, speculative.py:152-195)
pinned by the mathematics of its draws, not by a restatement of its code.

* The resample after a rejection follows normalize(max(0, t - d))
  (speculative.py:171-182), or t when that residual sums to <= 1e-6.
* The bonus follows the top-p filtered target row K (speculative.py:57-84);
  the keep set here comes from torch.sort + the shifted cumsum, the
  reference's own formulation, not from the oracle's sort-free rule.
* A rejection at the last draft position also appends a bonus (the
  reference's `num_accepted == self.k` branch, speculative.py:188).
* Draws never return a zero-weight token, at u = 0 or u just below 1.

Each chi-square test also checks its own power: the same draws must reject a
plausible wrong distribution (draft-minus-target residual, unfiltered target).
"""
import numpy as np
import pytest
import torch
from scipy import stats

from oracle import oracle as O

N_DRAWS = 40000


def _topp_keep_sorted(p: np.ndarray, top_p: float) -> np.ndarray:
    """speculative.py:67-81 evaluated with torch: sort, softmax-cumsum, shift."""
    x = torch.from_numpy(p.astype(np.float64))
    sp, si = torch.sort(x, descending=True)
    remove = torch.cumsum(sp, 0) > top_p
    remove[1:] = remove[:-1].clone()
    remove[0] = False
    keep = torch.ones_like(x, dtype=torch.bool)
    keep[si[remove]] = False
    return keep.numpy()


def _chi2_p(draws: np.ndarray, expected: np.ndarray) -> float:
    V = expected.size
    counts = np.bincount(draws, minlength=V)
    support = expected > 0
    assert counts[~support].sum() == 0, "a draw landed on a zero-probability token"
    exp = expected[support] / expected[support].sum() * draws.size
    return float(stats.chisquare(counts[support], exp).pvalue)


def _rows(p, B):
    return np.ascontiguousarray(np.broadcast_to(p, (B,) + p.shape)).astype(np.float32)


def _case(V=10, seed=0):
    rng = np.random.default_rng(seed)
    t = rng.dirichlet(np.ones(V) * 0.7, size=2).astype(np.float32)  # rows 0 (pos 0), 1 (bonus)
    d = rng.dirichlet(np.ones(V) * 0.7, size=1).astype(np.float32)
    return t, d


def test_rejection_at_last_position_appends_bonus():
    """K = 4, drafts certain at 0..2, impossible at 3: 5 tokens, rate 5/4."""
    B, K, V = 3, 4, 16
    t = np.zeros((B, K + 1, V), np.float32)
    d = np.zeros((B, K, V), np.float32)
    tok = np.full((B, K), 7, np.int32)
    for i in range(K):
        d[:, i, 7] = 1.0
        t[:, i, 7 if i < K - 1 else 3] = 1.0
    t[:, K, 9] = 1.0
    U = np.random.default_rng(1).random((B, K + 2)).astype(np.float32)
    n, ne, toks = O.python_verify(t, d, tok, U, 0.9)
    assert (n, ne) == (K - 1, K + 1)
    assert toks.tolist() == [[7, 7, 7, 3, 9]] * B
    # a rejection earlier than K - 1 emits no bonus
    t2 = t.copy()
    t2[:, 1, 7], t2[:, 1, 3] = 0.0, 1.0
    n, ne, toks = O.python_verify(t2, d, tok, U, 0.9)
    assert (n, ne) == (1, 2)
    assert toks.tolist() == [[7, 3, -1, -1, -1]] * B
    # full acceptance: K drafts and the bonus
    t3 = t.copy()
    t3[:, K - 1, 3], t3[:, K - 1, 7] = 0.0, 1.0
    n, ne, toks = O.python_verify(t3, d, tok, U, 0.9)
    assert (n, ne) == (K, K + 1)
    assert toks.tolist() == [[7, 7, 7, 7, 9]] * B


@pytest.mark.parametrize("top_p", [0.5, 0.9, 1.0])
def test_resample_and_bonus_follow_their_distributions(top_p):
    """K = 1 with a forced lock-step rejection at position 0 = K - 1: every row
    draws one resample from row 0's residual and one bonus from row 1."""
    V = 10
    t, d = _case(V, seed=3)
    B = N_DRAWS
    tp = _rows(t, B)[:, :, :]
    dp = _rows(d, B)
    tok = np.zeros((B, 1), np.int32)
    tok[:, 0] = int(np.argmax(d[0] - t[0]))  # q < p there: the ratio is < 1
    U = np.random.default_rng(5).random((B, 3)).astype(np.float32)
    U[0, 0] = 0.999999  # one certain rejection makes n = 0 for the batch
    n, ne, toks = O.python_verify(tp, dp, tok, U, top_p)
    assert (n, ne) == (0, 2)
    resid = np.maximum(t[0].astype(np.float64) - d[0], 0.0)
    p_res = _chi2_p(toks[:, 0], resid)
    keep = _topp_keep_sorted(t[1], top_p)
    bonus = np.where(keep, t[1].astype(np.float64), 0.0)
    p_bon = _chi2_p(toks[:, 1], bonus)
    assert p_res > 1e-4 and p_bon > 1e-4, (p_res, p_bon)
    # power: the same draws reject the plausible wrong answers
    wrong_res = np.maximum(d[0].astype(np.float64) - t[0], 0.0) + 1e-3
    assert stats.chisquare(np.bincount(toks[:, 0], minlength=V),
                           wrong_res / wrong_res.sum() * B).pvalue < 1e-6
    if top_p < 1.0:
        unfiltered = t[1].astype(np.float64)
        assert stats.chisquare(np.bincount(toks[:, 1], minlength=V),
                               unfiltered / unfiltered.sum() * B).pvalue < 1e-6


def test_zero_residual_falls_back_to_target():
    """d >= t everywhere at the rejected position: the residual sums to 0 <=
    1e-6, so the resample follows t itself (speculative.py:177-180)."""
    V = 8
    t, _ = _case(V, seed=7)
    B = N_DRAWS
    tp = _rows(t, B)
    d0 = t[0].copy()
    d0[2] = np.float32(0.9)  # q > p at the drafted token: ratio < 1
    dp = _rows(d0[None, :], B)
    tok = np.full((B, 1), 2, np.int32)
    U = np.random.default_rng(6).random((B, 3)).astype(np.float32)
    U[0, 0] = 0.999999
    n, ne, toks = O.python_verify(tp, dp, tok, U, 1.0)
    assert n == 0
    assert O.py_sample_adjusted(t[0], d0, 0.5)[1]  # the fallback branch
    assert _chi2_p(toks[:, 0], t[0].astype(np.float64)) > 1e-4


def test_draws_never_return_zero_weight_tokens():
    """u = 0 and u = 1 - 2^-24 on rows whose first and last tokens are filtered
    out (top-p) or carry no residual mass."""
    V = 12
    p = np.full(V, 0.001, np.float32)
    p[4], p[6] = 0.6, 0.389
    p /= p.sum()
    keep = _topp_keep_sorted(p, 0.5)
    assert not keep[0] and not keep[V - 1]
    for u in (0.0, np.nextafter(np.float32(1), np.float32(0))):
        w = np.where(keep, p, 0).astype(np.float32)
        assert keep[O.sample_weights(w, u)]
        assert keep[O.sample_filtered(p, u, 0.5, 0)]
    t = np.zeros(V, np.float32)
    t[3], t[5] = 0.5, 0.5
    d = np.full(V, 1.0 / V, np.float32)
    for u in (0.0, np.nextafter(np.float32(1), np.float32(0))):
        tok, fb = O.py_sample_adjusted(t, d, u)
        assert not fb and tok in (3, 5)
    assert O.py_sample_adjusted(t, d, 0.0)[0] == 3
    assert O.py_sample_adjusted(t, d, np.nextafter(np.float32(1), np.float32(0)))[0] == 5


class _Peak:
    """CPU stub runner: logits 50 on token fn(t) at position t, 0 elsewhere."""

    def __init__(self, fn, V):
        self.fn, self.V = fn, V

    def forward(self, ids, kv=None):
        B, T = ids.shape
        out = torch.zeros(B, T, self.V)
        for t in range(T):
            out[:, t, self.fn(t)] = 50.0
        return out


def test_cpu_chain_step_quirks():
    """oracle.speculative_cpu.chain_step (the CPU path of the chain step): the
    reference's emitted tokens for forced outcomes."""
    from oracle.speculative_cpu import chain_step

    V, K, T0 = 64, 4, 6
    ids = torch.zeros(2, T0, dtype=torch.long)
    draft = _Peak(lambda t: 7, V)
    g = torch.Generator().manual_seed(0)
    last = _Peak(lambda t: 7 if t < T0 + K - 2 else (3 if t == T0 + K - 2 else 9), V)
    toks, n = chain_step(draft, last, ids, K, generator=g)
    assert n == K + 1 and toks.tolist() == [[7, 7, 7, 3, 9]] * 2
    full = _Peak(lambda t: 7 if t < T0 + K - 1 else 9, V)
    toks, n = chain_step(draft, full, ids, K, generator=g)
    assert n == K + 1 and toks.tolist() == [[7, 7, 7, 7, 9]] * 2
    early = _Peak(lambda t: 3 if t == T0 else 7, V)
    toks, n = chain_step(draft, early, ids, K, generator=g)
    assert n == 2 and toks.tolist() == [[7, 3]] * 2


def test_cpu_chain_step_random_runners():
    """Small random-init runners: the emitted prefix is the drafted prefix."""
    from cudaforge_amd.runners import DecoderRunner
    from oracle.speculative_cpu import chain_step

    V, K = 500, 4
    tgt = DecoderRunner(V, 64, 2, 2, 32, seed=1)
    drf = DecoderRunner(V, 32, 1, 1, 32, seed=2)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, V, (3, 20), generator=g)
    toks, n = chain_step(drf, tgt, ids, K, generator=g)
    assert 1 <= n <= K + 1 and toks.shape == (3, n)
    assert bool(((toks >= 0) & (toks < V)).all())
