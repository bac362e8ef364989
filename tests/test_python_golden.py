"""CPU tier: the python-mode oracle replayed on the reference's own run.

tests/golden/python_engine.* record what the reference's
``cudaforge/speculative.py`` ``SpeculativeEngine.step`` did
(tests/golden/make_python_golden.py ran it in the build container with
fed uniforms): per step, the drafted tokens, p_draft and the ratio of every
acceptance test, the emitted tokens, the weights each multinomial received
and the result fields.  The oracle is fed the same probabilities (torch's
CPU softmax, the reference's own op, checked bit for bit against the
recorded p_draft and ratios) and the same uniforms:

* accepted count, emitted count and the accepted prefix: exact;
* resample and bonus ids: exact wherever the uniform is not within rounding
  of a CDF boundary (the draws stand in for torch.multinomial with the same
  fed-uniform inverse CDF);
* the weights those draws use: within 1e-6 of the reference's normalised
  multinomial weights, with the same top-p keep sets away from the threshold
  and the same residual fallback.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.golden import python_engine as G

CASES = G.load(kinds=("random", "kat"))


def reference_probs(case, s):
    """softmax(logits / T) as the reference computes it (speculative.py:118, :145)."""
    T = max(case.temperature, 1e-5)
    tp = torch.softmax(torch.from_numpy(case.target_logits[s]) / T, dim=-1)
    dp = torch.softmax(torch.from_numpy(case.draft_logits[s]) / T, dim=-1)
    return tp, dp


def check_reference_probs(case, s, tp, dp):
    """The replayed probabilities are the reference's, bit for bit, at every
    acceptance test it ran."""
    st = case.steps[s]
    tok = torch.from_numpy(st["draft_tokens"])
    for i in range(st.rec["n_tests"]):
        p_draft = dp[:, i].gather(-1, tok[:, i:i + 1])
        q_target = tp[:, i].gather(-1, tok[:, i:i + 1])
        assert np.array_equal(p_draft.reshape(-1).numpy(), st["p_draft"][i])
        ratio = torch.minimum(torch.ones_like(q_target), q_target / (p_draft + 1e-8))
        assert np.array_equal(ratio.reshape(-1).numpy(), st["ratio"][i])


def _keep_diff_at_threshold(p, keep_ref, keep_orc, top_p):
    """Tokens kept by one rule and not the other must sit at the threshold:
    the mass strictly above them within 1e-5 of top_p."""
    diff = np.flatnonzero(keep_ref != keep_orc)
    p64 = p.astype(np.float64)
    for j in diff:
        above = p64[p64 > p64[j]].sum()
        assert abs(above - top_p) < 1e-5, f"keep sets differ away from the threshold at {j}"
    return diff.size


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_oracle_replays_reference_steps(case):
    compared = total = 0
    for s, st in enumerate(case.steps):
        assert st.exception is None
        tp, dp = reference_probs(case, s)
        check_reference_probs(case, s, tp, dp)
        tok = st["draft_tokens"].astype(np.int32)
        n, ne, out = O.python_verify(tp.numpy(), dp.numpy(), tok, st.uniforms(), case.top_p)
        n_ref = st.n_accepted_drafts
        assert n == n_ref, f"step {s}: accepted {n}, reference {n_ref}"
        assert ne == st.rec["num_accepted"]
        acc = st["accepted_tokens"]
        assert acc.shape == (case.B, ne)
        assert np.array_equal(acc[:, :n], tok[:, :n])
        assert np.array_equal(out[:, :n], tok[:, :n])
        for col, kind, ids, ok in G.final_columns(st, n):
            assert np.array_equal(acc[:, col], ids)
            total += ids.size
            compared += int(ok.sum())
            assert np.array_equal(out[ok, col], ids[ok]), f"step {s} {kind} draw"
    assert compared >= 0.9 * total


@pytest.mark.parametrize("case", [c for c in CASES if c.B * c.V <= 65536],
                         ids=[c.name for c in CASES if c.B * c.V <= 65536])
def test_oracle_draw_weights_match_reference(case):
    """The distributions the oracle draws from are the ones the reference
    handed to torch.multinomial (speculative.py:171-182, :57-84)."""
    fallbacks = 0
    for s, st in enumerate(case.steps):
        tp, dp = reference_probs(case, s)
        tp, dp = tp.numpy(), dp.numpy()
        n = st.n_accepted_drafts
        for f, kind in enumerate(st.rec["final_kinds"]):
            w_ref = st["final_weights"][f].astype(np.float64)
            for b in range(case.B):
                ref = w_ref[b] / w_ref[b].sum()
                if kind == "resample":
                    w, fb = O.py_residual_weights(tp[b, n], dp[b, n])
                    if fb:  # the reference drew from the target row itself (:177-180)
                        assert np.array_equal(st["final_weights"][f][b], tp[b, n])
                        fallbacks += 1
                    w = w.astype(np.float64) / w.astype(np.float64).sum()
                else:
                    assert st.rec["bonus_args"][0] == [max(case.temperature, 1e-5), case.top_p]
                    w = O.py_bonus_weights(tp[b, case.K], case.top_p).astype(np.float64)
                    if _keep_diff_at_threshold(tp[b, case.K], ref > 0, w > 0, case.top_p):
                        continue
                    assert np.array_equal(ref > 0, w > 0)
                assert np.abs(w - ref).max() <= 1e-6, f"step {s} row {b} {kind}"
    if case.name == "kat_fallback":
        assert fallbacks == case.B


def test_zero_target_probability_rejects_in_python_mode_and_accepts_in_cpp_mode():
    """u = 0 at a drafted token whose target probability is exactly 0: the
    python rule u < min(1, q / (p + 1e-8)) rejects (speculative.py:166; the
    reference's own run rejected), the cpp rule u <= ratio accepts
    (speculative.cpp:71-74)."""
    case = next(c for c in CASES if c.name == "kat_zero_target")
    st = case.steps[0]
    tp, dp = (x.numpy() for x in reference_probs(case, 0))
    tok = st["draft_tokens"].astype(np.int32)
    assert tp[0, 0, tok[0, 0]] == 0.0 and st["acc_u"][0, 0] == 0.0
    assert st.n_accepted_drafts == 0
    n, ne, _ = O.python_verify(tp, dp, tok, st.uniforms(), case.top_p)
    assert n == 0
    cpp = O.chain_verify(tp, dp, tok, np.zeros((case.B, case.K + 1), np.float32))
    assert cpp["accept_len"][0] >= 1


def test_u_on_the_ratio_rejects():
    """u equal to the reference's own ratio rejects; one ulp below accepts."""
    case = next(c for c in CASES if c.name == "kat_u_at_ratio")
    for s, (i_star, b_star) in enumerate(case.meta["plan"]):
        st = case.steps[s]
        u, r = st["acc_u"][b_star, i_star], st["ratio"][i_star][b_star]
        accepted = st.n_accepted_drafts > i_star
        assert accepted == bool(u < r)
        tp, dp = (x.numpy() for x in reference_probs(case, s))
        n, _, _ = O.python_verify(tp, dp, st["draft_tokens"].astype(np.int32), st.uniforms(),
                                  case.top_p)
        assert n == st.n_accepted_drafts
    kinds = [(s % 3) for s in range(len(case.steps))]
    assert [case.steps[s].n_accepted_drafts > case.meta["plan"][s][0]
            for s in range(len(case.steps))] == [k == 1 for k in kinds]


def test_reference_step_telemetry():
    """Result fields of the reference run, as the drop-in must reproduce them:
    num_accepted counts the resampled or bonus token, a rejection at K - 1
    adds the bonus (K + 1 tokens), acceptance_rate = num_accepted / K,
    lifetime totals accumulate (speculative.py:184-217)."""
    for case in CASES:
        tot = 0
        for s, st in enumerate(case.steps):
            n = st.n_accepted_drafts
            ne = st.rec["num_accepted"]
            assert ne == n + 1 + (1 if n == case.K - 1 else 0)
            assert st.rec["acceptance_rate"] == ne / case.K
            tot += ne
            assert st.rec["total_accepted_tokens"] == tot
            assert st.rec["total_draft_tokens"] == case.K * (s + 1)
    degenerate = {c.name: c for c in G.load(kinds=("degenerate",))}
    for name in ("k0_b1", "k0_b4"):
        st = degenerate[name].steps[0]
        assert st.exception == ["ValueError", "torch.cat(): expected a non-empty list of Tensors"]
        assert st.rec["target_calls"] == 0 and st.rec["total_accepted_tokens"] == 0
    st = degenerate["b0_k4"].steps[0]
    assert st.rec["num_accepted"] == 5 and st.rec["accepted_shape"] == [0, 5]
