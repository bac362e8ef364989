"""GPU tier: the drop-in ``cudaforge_amd.speculative.SpeculativeEngine`` end to
end, against ``cudaforge/speculative.py:27-217``.

The chain step runs with random-init fp32 runners at the reference CPU
step's shapes (target 4 layers / d 512 / 8 heads of 64, draft 1 layer /
d 256 / 4 heads, vocabulary 32000, prompt 128, K = 4, T = 1.0) at B = 1 and
B = 64, in both verify modes.  Each step's kernel inputs are rebuilt from
what the runners returned; the probabilities the kernel used are checked
against a float64 softmax (1e-6), and the accept count, the emitted ids and
the telemetry against the oracle fed those probabilities and the uniforms
the step drew.  Stub runners force the reference's quirks: a rejection at the
last position appends a bonus (K + 1 tokens), K = 0 raises the reference's
ValueError before the target runs.  tests/test_python_golden_gpu.py replays
the reference's own recorded steps.
"""
import numpy as np
import pytest
import torch
from scipy import stats

from oracle import oracle as O
from cudaforge_amd.runners import draft_runner, target_runner
from cudaforge_amd.speculative import SpeculativeBatchResult, SpeculativeEngine
from cudaforge_amd.verify import chain_verify

pytestmark = pytest.mark.gpu

V_C1, K_C1, PROMPT_C1 = 32000, 4, 128


class Recorder:
    """Duck-typed runner wrapper that keeps every call's ids and logits."""

    def __init__(self, runner):
        self.runner = runner
        self.calls = []

    def forward(self, input_ids, kv_cache_handles=None):
        out = self.runner.forward(input_ids, kv_cache_handles)
        self.calls.append((input_ids.clone(), out))
        return out


@pytest.fixture(scope="module")
def c1_runners(device):
    return target_runner(seed=1, device=device), draft_runner(seed=2, device=device)


def _check_step(eng, res, drec, trec, prompt, mode):
    K = eng.k
    B, T0 = prompt.shape
    ids_v, tlog = trec.calls[-1]
    assert torch.equal(ids_v[:, :T0], prompt)
    tok = ids_v[:, T0:]
    assert tok.shape == (B, K) and bool(((tok >= 0) & (tok < tlog.shape[-1])).all())
    dcalls = drec.calls[-K:]
    for i, (ids, _) in enumerate(dcalls):  # autoregressive draft inputs (speculative.py:113-123)
        assert torch.equal(ids, torch.cat([prompt, tok[:, :i]], dim=-1))
    dl = torch.stack([c[1][:, -1, :].float() for c in dcalls], dim=1)
    win = tlog[:, -(K + 1):, :].float()
    out = chain_verify(win, dl, tok.to(torch.int32), res.uniforms, input_kind="logits",
                       temperature=eng.temperature, top_p=eng.top_p, mode=mode,
                       return_probs=True)
    tp, dp = out.target_probs, out.draft_probs
    for p, x in ((tp, win), (dp, dl)):
        ref = torch.softmax(x.double() / eng.temperature, dim=-1)
        assert (p.double() - ref).abs().max().item() <= 1e-6
    tp, dp = tp.cpu().numpy(), dp.cpu().numpy()
    U = res.uniforms.cpu().numpy()
    tk = tok.to(torch.int32).cpu().numpy()
    got = res.accepted_tokens.cpu().numpy()
    if mode == "python":
        assert U.shape == (B, K + 2)
        n, ne, toks = O.python_verify(tp, dp, tk, U, eng.top_p)
        assert res.num_accepted == ne and got.shape == (B, ne)
        np.testing.assert_array_equal(got, toks[:, :ne])
        assert res.num_emitted_per_row is None
    else:
        assert U.shape == (B, K + 1)
        want = O.chain_verify(tp, dp, tk, U)
        w = int(want["num_emitted"].max())
        assert res.num_accepted == w and got.shape == (B, w)
        np.testing.assert_array_equal(got, want["tokens"][:, :w])
        np.testing.assert_array_equal(res.num_emitted_per_row.cpu().numpy(),
                                      want["num_emitted"])
    assert res.draft_tokens_generated == K
    assert res.acceptance_rate == res.num_accepted / K
    assert res.draft_latency_ms > 0 and res.target_latency_ms > 0
    return got


@pytest.mark.parametrize("mode", ["python", "cpp"])
def test_c1_chain_steps(device, c1_runners, mode):
    """Three successive steps at B = 1, each fed the previous step's tokens."""
    tgt, drf = c1_runners
    drec, trec = Recorder(drf), Recorder(tgt)
    gen = torch.Generator(device=device).manual_seed(11)
    eng = SpeculativeEngine(drec, trec, num_speculative_tokens=K_C1, temperature=1.0,
                            verify_mode=mode, generator=gen)
    assert (eng.k, eng.temperature, eng.top_p) == (K_C1, 1.0, 0.9)
    ids = torch.randint(0, V_C1, (1, PROMPT_C1), device=device,
                        generator=torch.Generator(device=device).manual_seed(3))
    total = 0
    for step in range(3):
        res = eng.step(ids)
        assert isinstance(res, SpeculativeBatchResult)
        got = _check_step(eng, res, drec, trec, ids, mode)
        total += res.num_accepted
        assert eng.total_draft_tokens == K_C1 * (step + 1)
        assert eng.total_accepted_tokens == total
        ids = torch.cat([ids, torch.from_numpy(got).to(device)], dim=-1)
    assert eng.get_aggregate_acceptance_rate() == total / (3 * K_C1)


@pytest.mark.parametrize("mode", ["python", "cpp"])
def test_c1_chain_step_batch64(device, c1_runners, mode):
    tgt, drf = c1_runners
    drec, trec = Recorder(drf), Recorder(tgt)
    gen = torch.Generator(device=device).manual_seed(12)
    eng = SpeculativeEngine(drec, trec, num_speculative_tokens=K_C1, temperature=1.0,
                            verify_mode=mode, generator=gen)
    ids = torch.randint(0, V_C1, (64, PROMPT_C1), device=device,
                        generator=torch.Generator(device=device).manual_seed(4))
    res = eng.step(ids)
    _check_step(eng, res, drec, trec, ids, mode)


class PeakRunner:
    """Stub runner: the logits at position t are 50 on token fn(t), 0 elsewhere."""

    def __init__(self, fn, V, device):
        self.fn, self.V, self.device = fn, V, device

    def forward(self, input_ids, kv_cache_handles=None):
        B, T = input_ids.shape
        out = torch.zeros(B, T, self.V, device=self.device)
        for t in range(T):
            out[:, t, self.fn(t)] = 50.0
        return out


def test_rejection_at_last_position_emits_bonus(device):
    """K = 4: drafts certain at 0..2, impossible at 3 -> 5 tokens, rate 1.25 (the
    reference's num_accepted == self.k branch, speculative.py:188-195)."""
    V, K, T0 = 64, 4, 6
    draft = PeakRunner(lambda t: 7, V, device)
    # window row i verifies position T0 - 1 + i
    target = PeakRunner(lambda t: 7 if t < T0 + K - 2 else (3 if t == T0 + K - 2 else 9),
                        V, device)
    eng = SpeculativeEngine(draft, target, num_speculative_tokens=K,
                            generator=torch.Generator(device=device).manual_seed(0))
    ids = torch.zeros(2, T0, dtype=torch.long, device=device)
    res = eng.step(ids)
    assert res.accepted_tokens.tolist() == [[7, 7, 7, 3, 9]] * 2
    assert res.num_accepted == 5 and res.acceptance_rate == 1.25
    assert eng.get_aggregate_acceptance_rate() == 1.25
    # cpp mode: a resample ends the row (speculative.cpp:84-91)
    eng_c = SpeculativeEngine(draft, target, num_speculative_tokens=K, verify_mode="cpp",
                              generator=torch.Generator(device=device).manual_seed(0))
    res = eng_c.step(ids)
    assert res.accepted_tokens.tolist() == [[7, 7, 7, 3]] * 2 and res.num_accepted == 4
    # full acceptance: K drafts and the bonus
    full = PeakRunner(lambda t: 7 if t < T0 + K - 1 else 9, V, device)
    res = SpeculativeEngine(draft, full, num_speculative_tokens=K).step(ids)
    assert res.accepted_tokens.tolist() == [[7, 7, 7, 7, 9]] * 2 and res.num_accepted == 5
    # an earlier rejection: no bonus
    early = PeakRunner(lambda t: 3 if t == T0 else 7, V, device)
    res = SpeculativeEngine(draft, early, num_speculative_tokens=K).step(ids)
    assert res.accepted_tokens.tolist() == [[7, 3]] * 2 and res.num_accepted == 2


def test_k_zero_raises_before_the_target_runs(device):
    """speculative.py:128: torch.cat of the empty draft list raises ValueError;
    the target never runs and the totals stay 0 (the reference's own run,
    tests/golden/python_engine.json cases k0_b1 / k0_b4)."""
    V = 32
    draft = Recorder(PeakRunner(lambda t: 5, V, device))
    target = Recorder(PeakRunner(lambda t: 5, V, device))
    eng = SpeculativeEngine(draft, target, num_speculative_tokens=0)
    with pytest.raises(ValueError, match="expected a non-empty list of Tensors"):
        eng.step(torch.zeros(1, 3, dtype=torch.long, device=device))
    assert not draft.calls and not target.calls
    assert eng.total_draft_tokens == 0 and eng.total_accepted_tokens == 0
    assert eng.get_aggregate_acceptance_rate() == 0.0


def _topp_keep_sorted(p: np.ndarray, top_p: float) -> np.ndarray:
    x = torch.from_numpy(p.astype(np.float64))
    sp, si = torch.sort(x, descending=True)
    remove = torch.cumsum(sp, 0) > top_p
    remove[1:] = remove[:-1].clone()
    remove[0] = False
    keep = torch.ones_like(x, dtype=torch.bool)
    keep[si[remove]] = False
    return keep.numpy()


@pytest.mark.parametrize("top_p", [0.5, 0.9, 1.0])
def test_sample_next_token_distribution(device, top_p):
    """_sample_next_token (speculative.py:57-84): 40,000 rows of one logit row
    follow the top-p filtered softmax (chi-square), never a filtered token."""
    V, B, T = 16, 40000, 0.8
    g = torch.Generator().manual_seed(5)
    row = torch.randn(V, generator=g) * 1.5
    eng = SpeculativeEngine(None, None, generator=torch.Generator(device=device).manual_seed(9))
    toks = eng._sample_next_token(row.to(device).expand(B, V).contiguous(), temperature=T,
                                  top_p=top_p)
    assert toks.shape == (B, 1) and toks.dtype == torch.int64
    p = torch.softmax(row.double() / T, 0).numpy()
    keep = _topp_keep_sorted(p, top_p)
    counts = np.bincount(toks[:, 0].cpu().numpy(), minlength=V)
    assert counts[~keep].sum() == 0
    exp = p[keep] / p[keep].sum() * B
    assert stats.chisquare(counts[keep], exp).pvalue > 1e-4
