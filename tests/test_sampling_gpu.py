"""GPU tier: the sampler (cfa_sample) against the oracle -- tokens bit-exact
given the probabilities the kernel used and the fed uniforms, probabilities
within 1e-6 abs of an fp64 softmax; the reference's own sampler test; a
chi-square check that independent draws of one row follow its distribution."""
import numpy as np
import pytest
import torch

from cudaforge_amd.sampling import (SamplingParams, expand_tree_level, fused_sampling_triton,
                                    launch_fused_sampling, sample)
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch_size", [1, 4, 16])
@pytest.mark.parametrize("vocab_size", [1024, 4096])
@pytest.mark.parametrize("temperature", [0.0, 0.7, 1.0])
def test_reference_sampler_kat(device, batch_size, vocab_size, temperature):
    """tests/unit/test_sampling_and_autotuner.py:6-26."""
    torch.manual_seed(42)
    logits = torch.randn((batch_size, vocab_size), dtype=torch.float16, device=device)
    logits[:, 42] += 10.0
    tokens = fused_sampling_triton(logits, temperature=temperature)
    assert tokens.shape == (batch_size,) and tokens.dtype == torch.int32
    assert torch.all(tokens == 42)      # the Triton sampler is an argmax at every T
    p = SamplingParams(logits=logits, batch_size=batch_size, vocab_size=vocab_size,
                       temperature=temperature)
    out = launch_fused_sampling(p)
    assert out.shape == (batch_size,) and out.dtype == torch.int32
    if temperature == 0.0:
        assert torch.all(out == 42)


def _logits(R, V, seed, sigma=2.0):
    g = torch.Generator().manual_seed(seed)
    return (sigma * torch.randn(R, V, generator=g)).float()


@pytest.mark.parametrize("R,V,draws,T", [(37, 1000, 3, 0.7), (3, 128256, 2, 0.7), (5, 4099, 1, 1.3)])
def test_multinomial_vs_oracle(device, R, V, draws, T):
    x = _logits(R, V, R + V)
    g = torch.Generator().manual_seed(7)
    u = torch.rand(R, draws, generator=g)
    u[0, 0] = 0.0                        # first index whatever its mass
    u[-1, -1] = float(np.float32(1.0) - np.float32(2.0 ** -24))  # may reach the V-1 fallback
    tok, probs = sample(x.to(device), temperature=T, draws=draws, uniforms=u.to(device),
                        return_probs=True)
    tok, probs = tok.cpu().numpy(), probs.cpu().numpy()
    ref = torch.softmax(x.double() / T, dim=-1).numpy()
    assert np.abs(probs - ref).max() <= 1e-6
    for r in range(R):
        for d in range(draws):
            assert tok[r, d] == O.sample_from_distribution(probs[r], float(u[r, d])), (r, d)
    assert tok[0, 0] == 0


@pytest.mark.parametrize("top_p,top_k", [(0.9, 0), (0.5, 0), (1.0, 50), (0.8, 20)])
def test_filtered_vs_oracle(device, top_p, top_k):
    R, V, T = 9, 5000, 0.8
    x = _logits(R, V, 11)
    u = torch.rand(R, 2, generator=torch.Generator().manual_seed(3))
    tok, probs = sample(x.to(device), mode="filtered", temperature=T, top_p=top_p, top_k=top_k,
                        draws=2, uniforms=u.to(device), return_probs=True)
    tok, probs = tok.cpu().numpy(), probs.cpu().numpy()
    for r in range(R):
        for d in range(2):
            assert tok[r, d] == O.sample_filtered(probs[r], float(u[r, d]), top_p, top_k), (r, d)


@pytest.mark.parametrize("R,V,k", [(5, 100, 1), (7, 4096, 2), (3, 128256, 8), (300, 2048, 3)])
def test_greedy_topk_vs_oracle(device, R, V, k):
    g = torch.Generator().manual_seed(R * V)
    x = torch.randint(-20, 20, (R, V), generator=g).float()  # many ties
    got = sample(x.to(device), mode="greedy", draws=k).cpu().numpy()
    assert (got == O.topk_greedy(x.numpy(), k)).all()


def test_draws_of_one_row_follow_its_distribution(device):
    p = np.array([0.05, 0.4, 0.1, 0.25, 0.2], np.float32)
    x = torch.from_numpy(np.log(p))[None, :]
    n = 40000
    tok = sample(x.to(device), draws=n, generator=torch.Generator(device=device).manual_seed(5))
    counts = np.bincount(tok.cpu().numpy().ravel(), minlength=5)
    expected = n * p.astype(np.float64)
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 18.47, (chi2, counts / n)  # chi-square(4) 99.9% quantile


def test_expand_tree_level(device):
    R, V = 12, 3000
    x = _logits(R, V, 5).to(device)
    u = torch.rand(R, 2, device=device)
    a = expand_tree_level(x, children=2, temperature=0.9, uniforms=u)
    b = sample(x, temperature=0.9, draws=2, uniforms=u)
    assert torch.equal(a, b) and a.shape == (R, 2)
    gr = expand_tree_level(x, children=2, mode="greedy").cpu().numpy()
    assert (gr == O.topk_greedy(x.cpu().numpy(), 2)).all()
