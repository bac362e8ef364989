"""GPU tier: tree verification (cfa_tree_verify) against the oracle's tree
walk (oracle/spec_oracle.c orc_tree_verify), bit-exact; and its reduction to
chain verification on a one-child chain."""
import numpy as np
import pytest
import torch

from cudaforge_amd import tree as T
from cudaforge_amd.verify import chain_verify, tree_verify
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _softmax64(x):
    x = x - x.max(-1, keepdims=True)
    e = np.exp(x)
    return e / e.sum(-1, keepdims=True)


def tree_case(seed, B, parents, V, sigma=2.0, noise=0.5, T_=0.7, eos_bias=False):
    """Per-node target/draft logits as in BASELINE configs[3]; node tokens are
    drawn from the parent's draft distribution."""
    rng = np.random.default_rng(seed)
    N = len(parents)
    tl = (sigma * rng.standard_normal((B, N, V))).astype(np.float32)
    dl = (tl + noise * rng.standard_normal((B, N, V))).astype(np.float32)
    if eos_bias:
        tl[..., 0] += 4.0
        dl[..., 0] += 4.0
    dp = _softmax64(dl.astype(np.float64) / T_)
    tok = np.zeros((B, N), np.int32)
    for b in range(B):
        for c in range(1, N):
            cdf = np.cumsum(dp[b, parents[c]])
            tok[b, c] = min(int(np.searchsorted(cdf, rng.random() * cdf[-1])), V - 1)
    U = rng.random((B, N + 1)).astype(np.float32)
    return tl, dl, tok, U


def _dev(device, *a):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(device) for x in a]


def _check(out, parents, tp, dp, tok, U, eos, greedy):
    B = tok.shape[0]
    for b in range(B):
        w = O.tree_verify(parents, tok[b], tp[b], dp[b] if dp is not None else tp[b], U[b],
                          eos=eos, greedy=greedy)
        L = len(w["path"])
        assert int(out.path_len[b]) == L, (b, w)
        assert out.path[b, :L].tolist() == list(w["path"]), b
        assert int(out.final[b]) == w["final"], b
        assert bool(out.eos[b]) == w["eos"], b
        emitted = [int(tok[b, n]) for n in w["path"][1:]]
        if not (L > 1 and emitted[-1] == eos):
            emitted.append(w["final"])
        assert int(out.num_emitted[b]) == len(emitted)
        assert out.tokens[b, : len(emitted)].tolist() == emitted, b


@pytest.mark.parametrize("mode", ["cpp", "greedy"])
@pytest.mark.parametrize("kind", ["binary63", "star", "random"])
def test_tree_probs_vs_oracle(device, mode, kind):
    rng = np.random.default_rng(7)
    if kind == "binary63":
        parents, B, V = T.binary_tree_parents(63), 8, 4096
    elif kind == "star":
        parents, B, V = np.array([-1] + [0] * 11, np.int32), 16, 3000
    else:
        N = 40
        parents, B, V = np.array([-1] + [int(rng.integers(0, i)) for i in range(1, N)],
                                 np.int32), 8, 2048
    tl, dl, tok, U = tree_case(11, B, parents, V, eos_bias=(kind == "random"))
    tp = _softmax64(tl.astype(np.float64) / 0.7).astype(np.float32)
    dp = _softmax64(dl.astype(np.float64) / 0.7).astype(np.float32)
    eos = 0 if kind == "random" else -1
    t_d, d_d, tok_d, U_d, p_d = _dev(device, tp, dp, tok, U, parents)
    out = tree_verify(t_d, d_d, p_d, tok_d, U_d, input_kind="probs", mode=mode, eos_token_id=eos)
    torch.cuda.synchronize()
    assert out.status.cpu().tolist() == [0] * B
    _check(_cpu(out), parents, tp, dp, tok, U, eos, mode == "greedy")


def _cpu(out):
    class C:
        pass
    c = C()
    for k in ("path", "path_len", "tokens", "num_emitted", "final", "eos", "status"):
        setattr(c, k, getattr(out, k).cpu())
    return c


def test_tree_logits_c4_shape(device):
    """BASELINE configs[3] shape for acceptance: 63-node binary tree,
    V = 128256, T = 0.7, fp32 logits; decisions vs the oracle fed the
    kernel's probabilities, softmax within 1e-6 of float64."""
    parents = T.binary_tree_parents(63)
    B, V = 4, 128256
    tl, dl, tok, U = tree_case(21, B, parents, V)
    t_d, d_d, tok_d, U_d, p_d = _dev(device, tl, dl, tok, U, parents)
    out = tree_verify(t_d, d_d, p_d, tok_d, U_d, input_kind="logits", temperature=0.7,
                      mode="cpp", return_probs=True)
    torch.cuda.synchronize()
    tp = out.target_probs.cpu().numpy()
    dp = out.draft_probs.cpu().numpy()
    c = _cpu(out)
    for b in range(B):
        for n in c.path[b][: int(c.path_len[b])].tolist():
            ref = _softmax64(tl[b, n].astype(np.float64) / 0.7)
            assert np.abs(tp[b, n] - ref).max() <= 1e-6
    _check(c, parents, tp, dp, tok, U, -1, False)


def test_tree_logits_c4_full_batch(device):
    """The whole tree-acceptance workload: B = 32 sequences, 63-node binary
    tree, V = 128256, T = 0.7, logits ~ 2 N(0,1) with N(0, 0.5) draft noise,
    node tokens drawn from the parent's draft softmax (inputs generated on the
    device).  Every sequence's path, tokens and final draw vs the oracle fed
    the kernel's probabilities; visited rows' softmax within 1e-6."""
    parents = T.binary_tree_parents(63)
    B, N, V, Tm = 32, 63, 128256, 0.7
    g = torch.Generator(device=device).manual_seed(2024)
    tl = 2.0 * torch.randn(B, N, V, device=device, generator=g)
    dl = tl + 0.5 * torch.randn(B, N, V, device=device, generator=g)
    par = torch.from_numpy(parents).to(device).long()
    rows = torch.softmax(dl[:, par[1:]] / Tm, dim=-1).reshape(-1, V)
    tok = torch.zeros(B, N, dtype=torch.int32, device=device)
    tok[:, 1:] = torch.multinomial(rows, 1, generator=g).view(B, N - 1).int()
    del rows
    U = torch.rand(B, N + 1, device=device, generator=g)
    p_d = torch.from_numpy(parents).to(device)
    out = tree_verify(tl, dl, p_d, tok, U, input_kind="logits", temperature=Tm, mode="cpp",
                      return_probs=True)
    torch.cuda.synchronize()
    c = _cpu(out)
    assert c.status.tolist() == [0] * B
    tp, dp = out.target_probs.cpu().numpy(), out.draft_probs.cpu().numpy()
    tl_c = tl.cpu().numpy()
    del out, tl, dl
    for b in range(B):
        for n in c.path[b][: int(c.path_len[b])].tolist():
            ref = _softmax64(tl_c[b, n].astype(np.float64) / Tm)
            assert np.abs(tp[b, n] - ref).max() <= 1e-6
    _check(c, parents, tp, dp, tok.cpu().numpy(), U.cpu().numpy(), -1, False)


def test_one_child_chain_equals_chain_verify(device):
    """A chain tree (parent = i - 1) is exactly verify_candidates."""
    B, K, V = 16, 6, 5000
    parents = T.chain_parents(K + 1)
    tl, dl, tok, U = tree_case(31, B, parents, V)
    tp = _softmax64(tl.astype(np.float64) / 0.7).astype(np.float32)
    dp = _softmax64(dl.astype(np.float64) / 0.7).astype(np.float32)
    t_d, d_d, tok_d, U_d, p_d = _dev(device, tp, dp, tok, U, parents)
    tv = tree_verify(t_d, d_d, p_d, tok_d, U_d, input_kind="probs", mode="cpp")
    # chain layout: target rows 0..K, draft rows 0..K-1, drafts = node tokens 1..K
    cv = chain_verify(t_d, d_d[:, :K], tok_d[:, 1:].contiguous(), U_d[:, : K + 1].contiguous(),
                      input_kind="probs", mode="cpp")
    torch.cuda.synchronize()
    assert torch.equal(tv.path_len - 1, cv.accept_len)
    assert torch.equal(tv.final, cv.final)
    assert torch.equal(tv.tokens[:, : K + 1], cv.tokens)


def test_uniform_stream_exhaustion_is_reported(device):
    parents = T.binary_tree_parents(15)
    B, V = 2, 512
    tl, dl, tok, U = tree_case(41, B, parents, V)
    tp = _softmax64(tl.astype(np.float64)).astype(np.float32)
    t_d, tok_d, U_d, p_d = _dev(device, tp, tok, U[:, :1].copy() * 0 + 0.999, parents)
    out = tree_verify(t_d, t_d.clone() * 2, p_d, tok_d, U_d, input_kind="probs", mode="cpp")
    torch.cuda.synchronize()
    assert out.status.cpu().tolist() == [1, 1]


@pytest.mark.parametrize("kind", ["probs", "logits"])
def test_large_vocab_rereads_rows(device, kind):
    """V = 140000: with 8 work-groups per sequence a share exceeds what the
    LDS holds, so the kernel that re-reads rows from HBM runs.  Decisions vs
    the oracle (fed the kernel's probabilities for logits input)."""
    parents = T.binary_tree_parents(15)
    B, V = 2, 140000
    tl, dl, tok, U = tree_case(51, B, parents, V)
    if kind == "probs":
        tp = _softmax64(tl.astype(np.float64) / 0.7).astype(np.float32)
        dp = _softmax64(dl.astype(np.float64) / 0.7).astype(np.float32)
        t_d, d_d, tok_d, U_d, p_d = _dev(device, tp, dp, tok, U, parents)
        out = tree_verify(t_d, d_d, p_d, tok_d, U_d, input_kind="probs", mode="cpp")
    else:
        t_d, d_d, tok_d, U_d, p_d = _dev(device, tl, dl, tok, U, parents)
        out = tree_verify(t_d, d_d, p_d, tok_d, U_d, input_kind="logits", temperature=0.7,
                          mode="cpp", return_probs=True)
    torch.cuda.synchronize()
    assert out.status.cpu().tolist() == [0] * B
    if kind == "logits":
        tp, dp = out.target_probs.cpu().numpy(), out.draft_probs.cpu().numpy()
    _check(_cpu(out), parents, tp, dp, tok, U, -1, False)
