"""GPU tier: the reference's own python-engine runs replayed on the HIP path.

tests/golden/python_engine.* record what ``cudaforge/speculative.py``'s
``SpeculativeEngine.step`` did for fed uniforms (written in the build
container by tests/golden/make_python_golden.py).  Each recorded step is
replayed three ways:

1. ``chain_verify`` in python mode fed the reference's probabilities (torch's
   CPU softmax, the reference's own op): the accepted count, the emitted count
   and the accepted prefix are exact on every step, the known answers with u
   exactly on the ratio and a zero target probability included.
2. ``chain_verify`` in python mode fed the logits (the kernel's own fused
   softmax, within 1e-6 of fp64): the same, except on steps where some
   acceptance test had its uniform within 1e-5 of its ratio.
3. The drop-in ``SpeculativeEngine.step`` over successive steps, with
   ``TableRunner`` runners on the GPU and the recorded draft tokens and
   uniforms fed through its ``_draw_draft`` and ``_rand`` hooks: the
   result fields, the emitted tokens and the lifetime totals.

Resample and bonus ids are compared wherever rounding cannot change them:
the uniform is not within 1e-5 of a CDF boundary of the reference's weights,
nor (bonus draws) within the mass of the tokens at the top-p threshold
(``bonus_comparable``).  K = 0 raises the reference's ValueError before the
target runs; an empty batch emits [0, K+1] tokens.
"""
import builtins

import numpy as np
import pytest
import torch

from cudaforge_amd.speculative import SpeculativeEngine
from cudaforge_amd.verify import chain_verify
from tests.golden import python_engine as G
from tests.golden.recipes import TableRunner

pytestmark = pytest.mark.gpu

CASES = G.load(kinds=("random", "kat"))
DEGENERATE = {c.name: c for c in G.load(kinds=("degenerate",))}


def _reference_probs(case, s):
    T = max(case.temperature, 1e-5)
    tp = torch.softmax(torch.from_numpy(case.target_logits[s]) / T, dim=-1)
    dp = torch.softmax(torch.from_numpy(case.draft_logits[s]) / T, dim=-1)
    return tp, dp


def _check_emitted(case, s, n, num_emitted, tokens):
    """n, per-row emitted counts and the [B, >= ne] emitted tokens of one step
    against the reference's record; returns (compared, total) final draws."""
    st = case.steps[s]
    n_ref, ne = st.n_accepted_drafts, st.rec["num_accepted"]
    assert n == n_ref, f"{case.name} step {s}: accepted {n}, reference {n_ref}"
    assert (np.asarray(num_emitted) == ne).all()
    acc = st["accepted_tokens"]
    assert np.array_equal(tokens[:, :n], acc[:, :n])
    compared = total = 0
    for f, (col, kind, ids, ok) in enumerate(G.final_columns(st, n)):
        if kind == "bonus":
            ok = G.bonus_comparable(case, s, ids, st["final_margin"][f])
        total += ids.size
        compared += int(ok.sum())
        assert np.array_equal(tokens[ok, col], ids[ok]), f"{case.name} step {s} {kind}"
    return compared, total


@pytest.mark.parametrize("input_kind", ["probs", "logits"])
@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_kernel_replays_reference_steps(device, case, input_kind):
    compared = total = steps = 0
    for s, st in enumerate(case.steps):
        if input_kind == "logits" and G.knife_edge(st):
            continue
        steps += 1
        if input_kind == "probs":
            t, d = (x.to(device) for x in _reference_probs(case, s))
        else:
            t = torch.from_numpy(case.target_logits[s]).to(device)
            d = torch.from_numpy(case.draft_logits[s]).to(device)
        tok = torch.from_numpy(st["draft_tokens"].astype(np.int32)).to(device)
        u = torch.from_numpy(st.uniforms()).to(device)
        out = chain_verify(t, d, tok, u, input_kind=input_kind, temperature=case.temperature,
                           top_p=case.top_p, mode="python")
        torch.cuda.synchronize()
        n = int(out.accept_len[0].item())
        assert (out.accept_len.cpu().numpy() == n).all()
        c, tt = _check_emitted(case, s, n, out.num_emitted.cpu().numpy(), out.tokens.cpu().numpy())
        compared, total = compared + c, total + tt
    assert steps > 0 or case.name == "kat_u_at_ratio"
    assert compared >= 0.6 * total


class FedEngine(SpeculativeEngine):
    """The drop-in engine with the reference run's draws fed in: the recorded
    draft tokens (speculative.py:119) and the step's uniforms [B, K+2]."""

    def __init__(self, case, *args, **kw):
        super().__init__(*args, **kw)
        self.case, self.s, self.j = case, 0, 0

    def _draw_draft(self, probs):
        col = self.case.steps[self.s]["draft_tokens"][:, self.j:self.j + 1]
        self.j += 1
        return torch.from_numpy(np.ascontiguousarray(col)).to(probs.device)

    def _rand(self, *shape, device):
        st = self.case.steps[self.s]
        u = st.uniforms()
        assert tuple(shape) == u.shape
        self.s, self.j = self.s + 1, 0
        return torch.from_numpy(u).to(device)


DROPIN = [c for c in CASES if not any(G.knife_edge(st) for st in c.steps)]


@pytest.mark.parametrize("case", DROPIN, ids=[c.name for c in DROPIN])
def test_dropin_step_replays_reference(device, case):
    draft = TableRunner(case.draft_logits, draft=True, device=device)
    target = TableRunner(case.target_logits, draft=False, device=device)
    eng = FedEngine(case, draft, target, num_speculative_tokens=case.K,
                    temperature=case.temperature, top_p=case.top_p)
    ids = torch.zeros(case.B, 3, dtype=torch.long, device=device)
    for s, st in enumerate(case.steps):
        res = eng.step(ids)
        rec = st.rec
        assert res.num_accepted == rec["num_accepted"]
        assert res.draft_tokens_generated == rec["draft_tokens_generated"] == case.K
        assert res.acceptance_rate == rec["acceptance_rate"]
        assert list(res.accepted_tokens.shape) == rec["accepted_shape"]
        assert res.accepted_tokens.dtype == torch.int64
        acc = res.accepted_tokens.cpu().numpy()
        _check_emitted(case, s, st.n_accepted_drafts, [acc.shape[1]], acc)
        assert eng.total_draft_tokens == rec["total_draft_tokens"]
        assert eng.total_accepted_tokens == rec["total_accepted_tokens"]
        assert eng.get_aggregate_acceptance_rate() == rec["aggregate_rate"]
        assert draft.calls == case.K * (s + 1) and target.calls == s + 1
        # the target received the prompt and the drafted tokens (speculative.py:138)
        assert np.array_equal(target.inputs[-1][:, 3:].numpy(), st["draft_tokens"])


@pytest.mark.parametrize("name", ["k0_b1", "k0_b4"])
def test_dropin_k_zero_matches_reference(device, name):
    case = DEGENERATE[name]
    st = case.steps[0]
    draft = TableRunner(case.draft_logits, draft=True, device=device)
    target = TableRunner(case.target_logits, draft=False, device=device)
    eng = FedEngine(case, draft, target, num_speculative_tokens=0)
    exc_type, msg = st.exception
    with pytest.raises(getattr(builtins, exc_type)) as ei:
        eng.step(torch.zeros(case.B, 3, dtype=torch.long, device=device))
    assert type(ei.value).__name__ == exc_type and str(ei.value) == msg
    assert draft.calls == st.rec["draft_calls"] and target.calls == st.rec["target_calls"] == 0
    assert eng.total_draft_tokens == st.rec["total_draft_tokens"] == 0
    assert eng.total_accepted_tokens == st.rec["total_accepted_tokens"] == 0
    assert eng.get_aggregate_acceptance_rate() == st.rec["aggregate_rate"]


def test_dropin_empty_batch_matches_reference(device):
    case = DEGENERATE["b0_k4"]
    st = case.steps[0]
    draft = TableRunner(case.draft_logits, draft=True, device=device)
    target = TableRunner(case.target_logits, draft=False, device=device)
    eng = FedEngine(case, draft, target, num_speculative_tokens=case.K)
    res = eng.step(torch.zeros(0, 3, dtype=torch.long, device=device))
    assert res.num_accepted == st.rec["num_accepted"]
    assert list(res.accepted_tokens.shape) == st.rec["accepted_shape"]
    assert res.acceptance_rate == st.rec["acceptance_rate"]
    assert eng.total_accepted_tokens == st.rec["total_accepted_tokens"]
    assert eng.total_draft_tokens == st.rec["total_draft_tokens"]
    assert eng._sample_next_token(torch.zeros(0, 8, device=device)).shape == (0, 1)
