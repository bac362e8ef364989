"""GPU tier: python-mode draws of cfa_chain_verify (speculative.py:171-195) and
of the filtered sampler, on the HIP path.

The reference draws these with torch.multinomial, which cannot be fed
uniforms, so their ids are pinned in distribution: 40,000 draws per case,
chi-square against normalize(max(0, t - d)) (or t when that residual sums to
<= 1e-6) for the resample and against the top-p filtered target (keep set
from torch.sort + shifted cumsum) for the bonus.  The same draws are also
bit-exact with the oracle fed the same probabilities and uniforms.  Edge
uniforms (0 and 1 - 2^-24) never return a zero-weight token.
"""
import numpy as np
import pytest
import torch
from scipy import stats

from oracle import oracle as O
from cudaforge_amd.sampling import sample
from cudaforge_amd.verify import chain_verify

pytestmark = pytest.mark.gpu

N = 40000


def _keep_sorted(p: np.ndarray, top_p: float) -> np.ndarray:
    x = torch.from_numpy(p.astype(np.float64))
    sp, si = torch.sort(x, descending=True)
    remove = torch.cumsum(sp, 0) > top_p
    remove[1:] = remove[:-1].clone()
    remove[0] = False
    keep = torch.ones_like(x, dtype=torch.bool)
    keep[si[remove]] = False
    return keep.numpy()


def _chi2(draws, expected):
    counts = np.bincount(draws, minlength=expected.size)
    sup = expected > 0
    assert counts[~sup].sum() == 0, "a draw landed on a zero-probability token"
    return stats.chisquare(counts[sup], expected[sup] / expected[sup].sum() * draws.size).pvalue


def _dev(device, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in arrays]


def _run(device, t, d, tok, U, top_p):
    t_d, d_d, k_d, u_d = _dev(device, t, d, tok, U)
    out = chain_verify(t_d, d_d, k_d, u_d, input_kind="probs", mode="python", top_p=top_p)
    return out


@pytest.mark.parametrize("top_p", [0.5, 0.9, 1.0])
def test_resample_and_bonus_distribution(device, top_p):
    """K = 1, one certain rejection: n = 0 = K - 1 for the batch, so every row
    draws a resample from row 0's residual and a bonus from row 1."""
    V = 10
    rng = np.random.default_rng(3)
    t = rng.dirichlet(np.ones(V) * 0.7, size=2).astype(np.float32)
    d = rng.dirichlet(np.ones(V) * 0.7, size=1).astype(np.float32)
    tp = np.ascontiguousarray(np.broadcast_to(t, (N, 2, V)))
    dp = np.ascontiguousarray(np.broadcast_to(d, (N, 1, V)))
    tok = np.full((N, 1), int(np.argmax(d[0] - t[0])), np.int32)
    U = np.random.default_rng(5).random((N, 3)).astype(np.float32)
    U[0, 0] = 0.999999
    out = _run(device, tp, dp, tok, U, top_p)
    assert (out.accept_len.cpu() == 0).all() and (out.num_emitted.cpu() == 2).all()
    toks = out.tokens.cpu().numpy()
    n, ne, want = O.python_verify(tp, dp, tok, U, top_p)
    assert (n, ne) == (0, 2)
    np.testing.assert_array_equal(toks, want)
    np.testing.assert_array_equal(out.final.cpu().numpy(), toks[:, 1])
    assert _chi2(toks[:, 0], np.maximum(t[0].astype(np.float64) - d[0], 0.0)) > 1e-4
    keep = _keep_sorted(t[1], top_p)
    assert _chi2(toks[:, 1], np.where(keep, t[1].astype(np.float64), 0.0)) > 1e-4


def test_full_acceptance_bonus_distribution(device):
    """Ratio 1 everywhere: n = K for the batch, the bonus comes from row K."""
    V, K = 12, 2
    rng = np.random.default_rng(8)
    t = rng.dirichlet(np.ones(V), size=K + 1).astype(np.float32)
    tok = np.array([[1, 2]], np.int32).repeat(N, 0)
    t[0, 1], t[1, 2] = 0.5, 0.5  # q >= p at the drafts: ratio clamps to 1
    d = np.full((K, V), 0.01, np.float32)
    tp = np.ascontiguousarray(np.broadcast_to(t, (N, K + 1, V)))
    dp = np.ascontiguousarray(np.broadcast_to(d, (N, K, V)))
    U = np.random.default_rng(9).random((N, K + 2)).astype(np.float32)
    out = _run(device, tp, dp, tok, U, 0.7)
    assert (out.accept_len.cpu() == K).all() and (out.num_emitted.cpu() == K + 1).all()
    toks = out.tokens.cpu().numpy()
    np.testing.assert_array_equal(toks, O.python_verify(tp, dp, tok, U, 0.7)[2])
    keep = _keep_sorted(t[K], 0.7)
    assert _chi2(toks[:, K], np.where(keep, t[K].astype(np.float64), 0.0)) > 1e-4


def test_zero_residual_resamples_target(device):
    """d >= t: the residual sums to 0 <= 1e-6 and the resample follows t
    (speculative.py:177-180)."""
    V = 8
    rng = np.random.default_rng(7)
    t = rng.dirichlet(np.ones(V), size=3).astype(np.float32)
    d = t[:2].copy()
    d[0, 2] = 0.9
    tok = np.full((N, 2), 2, np.int32)
    tp = np.ascontiguousarray(np.broadcast_to(t, (N, 3, V)))
    dp = np.ascontiguousarray(np.broadcast_to(d, (N, 2, V)))
    U = np.random.default_rng(6).random((N, 4)).astype(np.float32)
    U[0, 0] = 0.999999
    out = _run(device, tp, dp, tok, U, 1.0)
    assert (out.accept_len.cpu() == 0).all() and (out.num_emitted.cpu() == 1).all()
    toks = out.tokens.cpu().numpy()
    np.testing.assert_array_equal(toks, O.python_verify(tp, dp, tok, U, 1.0)[2])
    assert _chi2(toks[:, 0], t[0].astype(np.float64)) > 1e-4


def test_edge_uniforms_skip_zero_weight_tokens(device):
    """u = 0 and u = 1 - 2^-24 on rows whose first and last tokens are filtered
    out (bonus, filtered sampler) or carry no residual (resample)."""
    V = 4096
    one_m = np.nextafter(np.float32(1), np.float32(0))
    p = np.full(V, 1e-6, np.float32)
    p[100], p[2000], p[3000] = 0.5, 0.3, 0.19
    p /= p.sum()
    keep = _keep_sorted(p, 0.6)
    assert not keep[0] and not keep[V - 1]
    # bonus (K = 0)
    tp = np.stack([p[None, :], p[None, :]])
    dp = np.zeros((2, 0, V), np.float32)
    tok = np.zeros((2, 0), np.int32)
    U = np.array([[0.0, 0.5], [one_m, 0.5]], np.float32)
    out = _run(device, tp, dp, tok, U, 0.6)
    toks = out.tokens.cpu().numpy()
    np.testing.assert_array_equal(toks, O.python_verify(tp, dp, tok, U, 0.6)[2])
    assert toks[0, 0] == 100 and keep[toks[1, 0]]
    # filtered sampler: the same keep rule
    s = sample(torch.from_numpy(p[None, :].repeat(2, 0)).to(device), mode="filtered",
               input_kind="probs", top_p=0.6, uniforms=torch.tensor([[0.0], [one_m]],
                                                                  device=device))
    assert s[:, 0].tolist() == [100, int(toks[1, 0])]
    # resample: residual mass only at tokens 7 and V - 9
    t = np.zeros((2, 2, V), np.float32)
    t[:, 0, 7], t[:, 0, V - 9] = 0.5, 0.5
    t[:, 1, 5] = 1.0
    d = np.full((2, 1, V), 1.0 / V, np.float32)
    d[:, 0, 3] = 0.9
    tok = np.full((2, 1), 3, np.int32)
    U = np.array([[0.5, 0.0, 0.5], [0.5, one_m, 0.5]], np.float32)
    out = _run(device, t, d, tok, U, 1.0)
    toks = out.tokens.cpu().numpy()
    np.testing.assert_array_equal(toks, O.python_verify(t, d, tok, U, 1.0)[2])
    assert toks[:, 0].tolist() == [7, V - 9] and toks[:, 1].tolist() == [5, 5]
