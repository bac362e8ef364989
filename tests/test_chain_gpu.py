"""GPU tier: the chain-verification kernels (cfa_chain_verify) against the
reference's golden vectors and the oracle.

Bar: accept lengths, emitted ids, final tokens and EOS flags bit-exact; the
fused softmax within 1e-6 abs of a float64 softmax.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import helpers as H
from tests.golden.recipes import c2_inputs, chain_case
from cudaforge_amd import SpeculativeConfig, SpeculativeEngine
from cudaforge_amd.verify import chain_verify

pytestmark = pytest.mark.gpu

SOFTMAX_ATOL = 1e-6


def _mt_stream(seed):
    seeds, draws = H.mt_stream()
    if np.uint64(seed) in seeds:
        return draws[list(seeds).index(np.uint64(seed))]
    from tests.test_oracle import mt19937_floats

    return mt19937_floats(seed, 256)


# --- the reference's own outputs through the compatibility engine ----------


@pytest.mark.parametrize("case", list(H.small_cases()), ids=lambda c: c[0])
@pytest.mark.parametrize("mode", ["cpp", "greedy"])
def test_compat_engine_matches_reference_golden(device, case, mode):
    name, seed, eos, tok, d, t, outs = case
    eng = SpeculativeEngine(SpeculativeConfig(rng_seed=seed), device=device)
    C, K = tok.shape
    got = dict(accepted=np.full((C, K), -1, np.int32), num_accepted=np.zeros(C, np.int32),
               final=np.zeros(C, np.int32), eos=np.zeros(C, np.int32))
    for c in range(C):
        if mode == "greedy":
            r = eng.verify_candidates_greedy(tok[c].tolist(), t[c].tolist(), eos)
        else:
            r = eng.verify_candidates(tok[c].tolist(), d[c].tolist(), t[c].tolist(), eos)
        got["accepted"][c, : r.num_accepted] = r.accepted_tokens
        got["num_accepted"][c] = r.num_accepted
        got["final"][c] = r.final_token
        got["eos"][c] = int(r.end_of_sequence)
    for k, v in outs[mode].items():
        np.testing.assert_array_equal(got[k], v, err_msg=f"{name} {mode} {k}")


@pytest.mark.parametrize("case", H.large_cases(), ids=lambda c: c["name"])
def test_compat_engine_matches_reference_golden_large(device, case):
    tok, d, t, eos = chain_case(case["seed"], case["calls"], case["K"], case["V"],
                                **case["kwargs"])
    assert H.digest(tok, d, t) == case["sha256"]
    eng = SpeculativeEngine(SpeculativeConfig(rng_seed=case["seed"]), device=device)
    for c in range(case["calls"]):
        r = eng.verify_candidates(tok[c], d[c], t[c], eos)
        n = case["out"]["num_accepted"][c]
        assert r.num_accepted == n
        assert r.accepted_tokens == case["out"]["accepted"][c][:n]
        assert r.final_token == case["out"]["final"][c]
        assert int(r.end_of_sequence) == case["out"]["eos"][c]


def test_reference_kats_through_gpu(device):
    # tests/unit/test_speculative.py:6-57
    cfg = SpeculativeConfig()
    cfg.gamma = 3
    eng = SpeculativeEngine(cfg, device=device)
    tp = [[0.0, 1.0, 0.0, 0.0, 0.0], [0.0, 0.0, 1.0, 0.0, 0.0], [0.0, 0.0, 0.0, 0.0, 1.0],
          [1.0, 0.0, 0.0, 0.0, 0.0]]
    r = eng.verify_candidates_greedy([1, 2, 3], tp, eos_token_id=0)
    assert r.num_accepted == 2 and r.accepted_tokens == [1, 2] and r.final_token == 4
    cfg.gamma = 2
    eng = SpeculativeEngine(cfg, device=device)
    r = eng.verify_candidates_greedy([1, 2], [[0.0, 1.0, 0.0], [0.0, 0.0, 1.0], [1.0, 0.0, 0.0]],
                                     eos_token_id=0)
    assert r.num_accepted == 2 and r.accepted_tokens == [1, 2] and r.final_token == 0
    assert r.end_of_sequence


# --- batched kernel vs oracle ----------------------------------------------


def _to_dev(device, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in arrays]


def _py_uniforms(U, seed=0):
    """[B, K+1] uniforms widened to python mode's [B, K+2] (one more column
    for the bonus that follows a rejection at the last position)."""
    extra = np.random.default_rng(seed).random((U.shape[0], 1)).astype(np.float32)
    return np.ascontiguousarray(np.concatenate([U, extra], axis=1))


def _check_vs_oracle(out, tp, dp, tok, U, eos, mode, top_p=1.0):
    if mode == "python":
        n, ne, toks = O.python_verify(tp, dp, tok, U, top_p)
        assert (out.accept_len.cpu().numpy() == n).all()
        assert (out.num_emitted.cpu().numpy() == ne).all()
        np.testing.assert_array_equal(out.tokens.cpu().numpy(), toks)
        last = toks[np.arange(toks.shape[0]), ne - 1]
        np.testing.assert_array_equal(out.final.cpu().numpy(), last)
        return
    want = O.chain_verify(tp, dp, tok, U, eos=eos, greedy=(mode == "greedy"))
    np.testing.assert_array_equal(out.accept_len.cpu().numpy(), want["accept_len"])
    np.testing.assert_array_equal(out.tokens.cpu().numpy(), want["tokens"])
    np.testing.assert_array_equal(out.num_emitted.cpu().numpy(), want["num_emitted"])
    np.testing.assert_array_equal(out.final.cpu().numpy(), want["final"])
    np.testing.assert_array_equal(out.eos.cpu().numpy(), want["eos"])


def _softmax64(x, T):
    x = torch.as_tensor(x, dtype=torch.float64) / T
    return torch.softmax(x, dim=-1)


@pytest.mark.parametrize("mode", ["cpp", "python", "greedy"])
@pytest.mark.parametrize("B,K,V", [(64, 8, 128256), (5, 3, 1001), (3, 0, 257), (2, 2, 1),
                                   (7, 1, 4096), (9, 5, 5001)])
def test_logits_path_matches_oracle(device, mode, B, K, V):
    T = 0.7
    tl, dl, tok, U = c2_inputs(seed=B * 1000 + K * 10 + V % 97, B=B, K=K, V=V, temperature=T)
    if mode == "python":
        U = _py_uniforms(U, seed=B + K)
    t_d, d_d, tok_d, U_d = _to_dev(device, tl, dl, tok, U)
    out = chain_verify(t_d, d_d, tok_d, U_d, input_kind="logits", temperature=T, mode=mode,
                       top_p=0.9, return_probs=True)
    torch.cuda.synchronize()
    tp = out.target_probs.cpu().numpy()
    err = (torch.from_numpy(tp).double() - _softmax64(tl, T)).abs().max().item()
    assert err <= SOFTMAX_ATOL, f"target softmax error {err}"
    if out.draft_probs is not None:
        dp = out.draft_probs.cpu().numpy()
        err = (torch.from_numpy(dp).double() - _softmax64(dl, T)).abs().max().item()
        assert err <= SOFTMAX_ATOL, f"draft softmax error {err}"
    else:
        dp = np.zeros((B, K, V), np.float32)
    _check_vs_oracle(out, tp, dp, tok, U, -1, mode, top_p=0.9)


@pytest.mark.parametrize("mode", ["cpp", "python", "greedy"])
def test_probs_path_matches_oracle(device, mode):
    tok, d, t, eos = chain_case(21, 48, 6, 3000, sigma=3.0, eos_bias=True)
    rng = np.random.default_rng(4)
    U = rng.random((48, 8 if mode == "python" else 7)).astype(np.float32)
    t_d, d_d, tok_d, U_d = _to_dev(device, t, d, tok, U)
    e = eos if mode != "python" else -1
    out = chain_verify(t_d, d_d, tok_d, U_d, input_kind="probs", mode=mode, eos_token_id=e,
                       top_p=0.8)
    _check_vs_oracle(out, t, d, tok, U, e, mode, top_p=0.8)


def test_uniforms_on_cdf_boundaries(device):
    """u placed exactly on (and one ulp below) sequential fp32 prefix sums."""
    B, K, V = 16, 0, 20000
    rng = np.random.default_rng(8)
    t = rng.random((B, 1, V)).astype(np.float32) ** 8
    t /= t.sum(-1, keepdims=True)
    U = np.zeros((B, 1), np.float32)
    for b in range(B):
        pref = np.cumsum(t[b, 0], dtype=np.float32)
        j = int(rng.integers(0, V))
        U[b, 0] = pref[j] if b % 2 == 0 else np.nextafter(pref[j], np.float32(0))
    d = np.zeros((B, 0, V), np.float32)
    tok = np.zeros((B, 0), np.int32)
    t_d, d_d, tok_d, U_d = _to_dev(device, t, d, tok, U)
    out = chain_verify(t_d, d_d, tok_d, U_d, input_kind="probs", mode="cpp")
    _check_vs_oracle(out, t, d, tok, U, -1, "cpp")


def test_uniforms_on_cdf_boundaries_of_first_tiles(device):
    """u on (and one ulp below) the prefix sums at the start of the row: the
    serially replayed leading tiles (indices 0..63), the first walked tile,
    the end of chunk 0 and the start of chunk 1 (1024 elements a chunk)."""
    js = [0, 1, 2, 15, 16, 31, 63, 64, 65, 79, 1023, 1024, 1040]
    B, K, V = 2 * len(js), 0, 5000
    rng = np.random.default_rng(12)
    t = rng.random((B, 1, V)).astype(np.float32) ** 8
    t /= t.sum(-1, keepdims=True)
    U = np.zeros((B, 1), np.float32)
    for b in range(B):
        pref = np.cumsum(t[b, 0], dtype=np.float32)
        j = js[b // 2]
        U[b, 0] = pref[j] if b % 2 == 0 else np.nextafter(pref[j], np.float32(0))
    d = np.zeros((B, 0, V), np.float32)
    tok = np.zeros((B, 0), np.int32)
    t_d, d_d, tok_d, U_d = _to_dev(device, t, d, tok, U)
    out = chain_verify(t_d, d_d, tok_d, U_d, input_kind="probs", mode="cpp")
    _check_vs_oracle(out, t, d, tok, U, -1, "cpp")
    got = out.tokens.cpu().numpy()[:, 0]
    for b in range(0, B, 2):  # u = s_j draws j exactly (speculative.cpp:19)
        assert got[b] == js[b // 2], (b, got[b])


def test_residual_fallback_equal_rows(device):
    tok, d, t, eos = chain_case(31, 32, 4, 500, equal=True)
    U = np.random.default_rng(2).random((32, 5)).astype(np.float32)
    t_d, d_d, tok_d, U_d = _to_dev(device, t, d, tok, U)
    out = chain_verify(t_d, d_d, tok_d, U_d, input_kind="probs", mode="cpp")
    _check_vs_oracle(out, t, d, tok, U, -1, "cpp")


def test_strided_window_of_larger_logits(device):
    """The target window is a view into [B, T, V] logits (speculative.py:144)."""
    B, K, V, Tlen = 4, 3, 1000, 11
    rng = np.random.default_rng(9)
    full = (2 * rng.standard_normal((B, Tlen, V))).astype(np.float32)
    dl = (full[:, Tlen - K - 1:Tlen - 1] + 0.5 * rng.standard_normal((B, K, V))).astype(np.float32)
    tok = rng.integers(0, V, (B, K)).astype(np.int32)
    U = rng.random((B, K + 1)).astype(np.float32)
    f_d, d_d, tok_d, U_d = _to_dev(device, full, dl, tok, U)
    win = f_d[:, -(K + 1):, :]
    out = chain_verify(win, d_d, tok_d, U_d, input_kind="logits", temperature=1.0, mode="cpp",
                       return_probs=True)
    tp = out.target_probs.cpu().numpy()
    dp = out.draft_probs.cpu().numpy()
    _check_vs_oracle(out, tp, dp, tok, U, -1, "cpp")


def test_out_of_range_token_is_rejected(device):
    B, K, V = 2, 2, 64
    t = np.full((B, K + 1, V), 1.0 / V, np.float32)
    d = np.full((B, K, V), 1.0 / V, np.float32)
    tok = np.array([[3, V + 5], [-1, 2]], np.int32)
    U = np.zeros((B, K + 1), np.float32)  # u = 0 would accept any valid token
    t_d, d_d, tok_d, U_d = _to_dev(device, t, d, tok, U)
    out = chain_verify(t_d, d_d, tok_d, U_d, input_kind="probs", mode="cpp")
    assert out.accept_len.cpu().tolist() == [1, 0]


def _chain_outputs(out):
    return [x.cpu().numpy() for x in (out.accept_len, out.tokens, out.num_emitted, out.final,
                                       out.eos)]


@pytest.mark.parametrize("case", ["c2", "all_accept", "eos_in_head", "small_v", "many_groups"])
def test_two_pass_statistics_match_one_pass(device, case):
    """cpp rules with logits read the rows of positions 0..2 first, and the
    rest only for sequences that accepted all three.  Every row is cut into
    the same slices in both passes, so the outputs are bit-identical to the
    one-pass run (return_probs=True reads every row), which the oracle checks
    in test_logits_path_matches_oracle.  The tail pass is the balanced one
    (stats_tail_kernel) for 16-byte rows and at most 4096 sequences, else the
    one-work-group-per-(row, slice) kernel: small_v (V % 4 != 0) and
    many_groups (B > 4096) take the latter."""
    T, eos = 0.7, -1
    if case == "small_v":
        tl, dl, tok, U = c2_inputs(seed=91, B=33, K=5, V=3001, temperature=T)
    elif case == "many_groups":
        tl, dl, tok, U = c2_inputs(seed=93, B=4100, K=4, V=256, temperature=T)
    else:
        tl, dl, tok, U = c2_inputs(seed=92, B=64, K=8, V=128256, temperature=T)
    if case == "all_accept":   # draft = target: every ratio is 1, every sequence needs its tail
        dl = tl[:, :-1].copy()
    if case == "eos_in_head":  # an accepted EOS at position 1 ends the walk in the head
        eos = int(tok[0, 1])
        tok[::2, 1] = eos
        U[::2, :2] = 0.0
    t_d, d_d, tok_d, U_d = _to_dev(device, tl, dl, tok, U)
    kw = dict(input_kind="logits", temperature=T, mode="cpp", eos_token_id=eos)
    one = chain_verify(t_d, d_d, tok_d, U_d, return_probs=True, **kw)
    two = chain_verify(t_d, d_d, tok_d, U_d, **kw)
    torch.cuda.synchronize()
    for a, b in zip(_chain_outputs(one), _chain_outputs(two)):
        np.testing.assert_array_equal(a, b)
    n = one.accept_len.cpu().numpy()
    if case == "all_accept":
        assert (n == tok.shape[1]).all()
    if case == "eos_in_head":
        assert (one.eos.cpu().numpy()[::2] == 1).all()
    if case == "c2":  # both outcomes present: sequences stopped in the head and ones that went on
        assert (n < 3).any() and (n >= 3).any()


def test_workspace_reuse_and_graph_replays(device):
    """The pipeline keeps state between its kernels in the workspace (the
    look-back words and cache counters, zeroed by the first statistics pass,
    the records, the jobs) and needs none of it to survive a call.  A call
    captured in a graph and replayed with new inputs copied in between, with
    eager calls on the same workspace interleaved, equals an eager call on a
    fresh workspace each time, and the outcomes differ between the input
    sets (so a replay that reused stale state would show)."""
    T, B, K, V = 0.7, 64, 8, 128256
    sets = [c2_inputs(seed=s, B=B, K=K, V=V, temperature=T) for s in (201, 202)]
    sets.append(sets[0][:1] + (sets[0][0][:, :-1].copy(),) + sets[0][2:])  # draft = target: all accept
    kw = dict(input_kind="logits", temperature=T, mode="cpp", eos_token_id=-1)
    t_d, d_d, tok_d, U_d = _to_dev(device, *sets[0])
    from cudaforge_amd.verify import chain_workspace_bytes
    ws = torch.empty(chain_workspace_bytes(B, K, V, "logits", "cpp"), dtype=torch.uint8, device=device)
    ws.fill_(0xA5)  # foreign contents
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):  # warm-up outside the capture, as torch requires
        chain_verify(t_d, d_d, tok_d, U_d, workspace=ws, **kw)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = chain_verify(t_d, d_d, tok_d, U_d, workspace=ws, **kw)
    seen = []
    for rep in range(7):
        src = sets[rep % 3]
        for dst, a in zip((t_d, d_d, tok_d, U_d), src):
            dst.copy_(torch.from_numpy(np.ascontiguousarray(a)))
        g.replay()
        torch.cuda.synchronize()
        got = _chain_outputs(out)
        ref = _chain_outputs(chain_verify(t_d, d_d, tok_d, U_d, **kw))
        for a, b in zip(got, ref):
            np.testing.assert_array_equal(a, b, err_msg=f"replay {rep}")
        if rep % 2:  # an eager call on the graph's workspace between replays
            eager = _chain_outputs(chain_verify(t_d, d_d, tok_d, U_d, workspace=ws, **kw))
            for a, b in zip(eager, ref):
                np.testing.assert_array_equal(a, b, err_msg=f"eager after replay {rep}")
        seen.append(got[0].copy())
    assert not np.array_equal(seen[0], seen[1]) and (seen[2] == K).all()
