"""CPU tier: pin the oracle (oracle/spec_oracle.c) before trusting it.

* against the golden vectors written from the reference's own compiled engine
  (tests/golden/make_golden.py; csrc/src/scheduler/speculative.cpp);
* against the reference's known-answer tests (tests/unit/test_speculative.py
  :6-57) restated on the oracle;
* live against oracle/_ref (the compiled reference) on fuzzed inputs, where
  it was built in this container;
* against closed forms and special cases of the inverse CDF, the residual
  fallback and the top-p rule.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import helpers as H
from tests.golden.recipes import chain_case


def oracle_one(greedy):
    def run(tok, d, t, eos, U):
        K = tok.size
        V = t.shape[-1]
        dd = d if K else np.zeros((0, V), np.float32)
        Uf = np.zeros(K + 1, np.float32)
        Uf[: U.size] = U
        out = O.chain_verify(t[None, : K + 1], dd[None], tok[None], Uf[None], eos=eos,
                             greedy=greedy)
        n = int(out["accept_len"][0])
        return list(out["tokens"][0, :n]), int(out["final"][0]), bool(out["eos"][0])
    return run


def stream_for(seed, n=4096):
    seeds, draws = H.mt_stream()
    idx = list(seeds).index(np.uint64(seed)) if np.uint64(seed) in seeds else None
    if idx is not None:
        return draws[idx]
    ref = O.ref_lib()
    if ref is None:
        pytest.skip("uniform stream for this seed needs oracle/_ref")
    return O.ref_uniforms(seed, n)


def mt19937_floats(seed, n):
    """std::mt19937 + uniform_real_distribution<float>(0,1) restated in numpy:
    MT19937 (Matsumoto & Nishimura 1998) 32-bit outputs, and libstdc++'s
    generate_canonical<float, 24> which, for a 32-bit engine, takes one output
    x and returns x * 2^-32 rounded to float (1.0 mapped below 1)."""
    mt = np.zeros(624, np.uint64)
    mt[0] = seed & 0xFFFFFFFF
    for i in range(1, 624):
        mt[i] = (1812433253 * (int(mt[i - 1]) ^ (int(mt[i - 1]) >> 30)) + i) & 0xFFFFFFFF
    mt = [int(x) for x in mt]
    out = []
    idx = 624
    for _ in range(n):
        if idx >= 624:
            for i in range(624):
                y = (mt[i] & 0x80000000) | (mt[(i + 1) % 624] & 0x7FFFFFFF)
                mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ (0x9908B0DF if y & 1 else 0)
            idx = 0
        y = mt[idx]
        idx += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9D2C5680
        y ^= (y << 15) & 0xEFC60000
        y ^= y >> 18
        f = np.float32(np.float32(y) / np.float32(4294967296.0))
        if f >= np.float32(1.0):
            f = np.nextafter(np.float32(1.0), np.float32(0.0))
        out.append(f)
    return np.array(out, np.float32)


# ---------------------------------------------------------------------------


def test_mt19937_fixture_matches_textbook_generator():
    seeds, draws = H.mt_stream()
    for s, row in zip(seeds, draws):
        np.testing.assert_array_equal(mt19937_floats(int(s), 700), row[:700])


@pytest.mark.parametrize("case", list(H.small_cases()), ids=lambda c: c[0])
@pytest.mark.parametrize("mode", ["cpp", "greedy"])
def test_oracle_matches_reference_golden(case, mode):
    name, seed, eos, tok, d, t, outs = case
    got = H.replay(oracle_one(mode == "greedy"), tok, d, t, eos, stream_for(seed),
                   mode == "greedy")
    want = outs[mode]
    for k in ("accepted", "num_accepted", "final", "eos"):
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"{name} {mode} {k}")


@pytest.mark.parametrize("case", H.large_cases(), ids=lambda c: c["name"])
def test_oracle_matches_reference_golden_large(case):
    tok, d, t, eos = chain_case(case["seed"], case["calls"], case["K"], case["V"],
                                **case["kwargs"])
    assert H.digest(tok, d, t) == case["sha256"], "input recipe stream changed"
    seeds, draws = H.mt_stream()
    stream = O.ref_uniforms(case["seed"], 4096) if O.ref_lib() else None
    if stream is None:
        stream = mt19937_floats(case["seed"], 64)
    got = H.replay(oracle_one(False), tok, d, t, eos, stream, False)
    for k, v in case["out"].items():
        np.testing.assert_array_equal(got[k], np.asarray(v), err_msg=k)


def test_reference_kat_greedy_partial():
    # tests/unit/test_speculative.py:23-37
    t = np.array([[0, 1, 0, 0, 0], [0, 0, 1, 0, 0], [0, 0, 0, 0, 1], [1, 0, 0, 0, 0]], np.float32)
    out = O.chain_verify(t[None], np.zeros((1, 3, 5), np.float32), np.array([[1, 2, 3]]),
                         np.zeros((1, 4), np.float32), eos=0, greedy=True)
    assert out["accept_len"][0] == 2
    assert list(out["tokens"][0, :2]) == [1, 2]
    assert out["final"][0] == 4


def test_reference_kat_greedy_full_acceptance_eos():
    # tests/unit/test_speculative.py:40-57
    t = np.array([[0, 1, 0], [0, 0, 1], [1, 0, 0]], np.float32)
    out = O.chain_verify(t[None], np.zeros((1, 2, 3), np.float32), np.array([[1, 2]]),
                         np.zeros((1, 3), np.float32), eos=0, greedy=True)
    assert out["accept_len"][0] == 2
    assert list(out["tokens"][0, :2]) == [1, 2]
    assert out["final"][0] == 0 and out["eos"][0] == 1


@pytest.mark.skipif(O.ref_lib() is None, reason="oracle/_ref not built (no reference mounted)")
@pytest.mark.parametrize("seed", range(20))
def test_oracle_matches_reference_live_fuzz(seed):
    rng = np.random.default_rng(1000 + seed)
    K = int(rng.integers(0, 9))
    V = int(rng.choice([1, 2, 7, 100, 3000]))
    kw = dict(sigma=float(rng.choice([0.5, 2.0, 6.0])), eos_bias=bool(rng.random() < 0.3),
              equal=bool(rng.random() < 0.2), zero_q=bool(rng.random() < 0.2))
    tok, d, t, eos = chain_case(2000 + seed, 8, K, V, **kw)
    for greedy in (False, True):
        want = O.ref_verify(2000 + seed, tok, d, t, eos, greedy=greedy)
        got = H.replay(oracle_one(greedy), tok, d, t, eos, O.ref_uniforms(2000 + seed, 4096),
                       greedy)
        for k in want:
            np.testing.assert_array_equal(got[k], want[k], err_msg=f"{k} greedy={greedy}")


# --- inverse CDF and residual: closed forms and special cases ---------------


def test_inverse_cdf_special_cases():
    p = np.array([0.0, 0.25, 0.25, 0.5], np.float32)
    assert O.sample_from_distribution(p, 0.0) == 0          # r = 0 returns index 0 (quirk)
    assert O.sample_from_distribution(p, 0.25) == 1          # boundary: r <= cumulative
    assert O.sample_from_distribution(p, np.nextafter(np.float32(0.25), np.float32(1))) == 2
    assert O.sample_from_distribution(p, 0.5) == 2
    assert O.sample_from_distribution(p, 0.999) == 3
    assert O.sample_from_distribution(np.array([0.1, 0.1], np.float32), 0.5) == 1  # falls through


def test_inverse_cdf_brute_force_float32():
    rng = np.random.default_rng(3)
    for _ in range(50):
        V = int(rng.integers(1, 300))
        p = rng.random(V).astype(np.float32)
        p /= p.sum()
        c = np.float32(0)
        prefix = []
        for x in p:
            c = np.float32(c + x)
            prefix.append(c)
        for r in list(rng.random(5).astype(np.float32)) + [prefix[int(rng.integers(0, V))]]:
            hit = [i for i, s in enumerate(prefix) if r <= s]
            assert O.sample_from_distribution(p, r) == (hit[0] if hit else V - 1)


def test_residual_fallback_and_normalisation():
    t = np.array([0.5, 0.5, 0.0], np.float32)
    d = np.array([0.5, 0.5, 0.0], np.float32)
    tok, fb = O.sample_adjusted(t, d, 0.7)
    assert fb and tok == 1                                     # sum 0 -> sample(target)
    t = np.array([0.6, 0.2, 0.2], np.float32)
    d = np.array([0.2, 0.6, 0.2], np.float32)
    tok, fb = O.sample_adjusted(t, d, 0.99)
    assert not fb and tok == 0                                 # residual is one-hot at 0


def test_ratio_quirks_cpp():
    # q = 0 -> ratio 0, u = 0 still accepts (r <= ratio), speculative.cpp:71-74
    t = np.full((1, 2, 4), 0.25, np.float32)
    d = np.zeros((1, 1, 4), np.float32)
    out = O.chain_verify(t, d, np.array([[2]]), np.array([[0.0, 0.5]], np.float32))
    assert out["accept_len"][0] == 1
    out = O.chain_verify(t, d, np.array([[2]]), np.array([[1e-7, 0.5]], np.float32))
    assert out["accept_len"][0] == 0


# --- top-p rule (speculative.py:67-81) ------------------------------------


@pytest.mark.parametrize("top_p,keep", [(0.6, [1, 1, 0]), (0.4, [1, 0, 0]), (0.5, [1, 1, 0]),
                                        (1.0, [1, 1, 1]), (0.0, [1, 0, 0])])
def test_topp_known_answers(top_p, keep):
    p = np.array([0.5, 0.3, 0.2], np.float32)
    assert list(O.topp_keep(p, top_p)) == [bool(k) for k in keep]


def test_topp_matches_sort_cumsum_rule():
    """The threshold form equals the reference's sort + shifted cumsum rule on
    distinct probabilities (ties aside): torch-CPU, fp64, no fed randomness."""
    import torch

    rng = np.random.default_rng(5)
    for _ in range(30):
        V = int(rng.integers(2, 500))
        logits = torch.from_numpy(rng.normal(0, 2, V))
        p = torch.softmax(logits, -1)
        top_p = float(rng.random())
        sp, si = torch.sort(p, descending=True)
        cum = torch.cumsum(sp, -1)
        remove = cum > top_p
        remove[1:] = remove[:-1].clone()
        remove[0] = False
        keep_ref = torch.ones(V, dtype=torch.bool)
        keep_ref[si[remove]] = False
        got = O.topp_keep(p.numpy().astype(np.float32), top_p)
        # compare where the fp64 and fp32 cumulative sums cannot straddle top_p
        margin = (cum - top_p).abs().min().item()
        if margin > 1e-6:
            assert np.array_equal(got, keep_ref.numpy())


def test_python_mode_lockstep_invariant():
    rng = np.random.default_rng(11)
    B, K, V = 6, 5, 50
    tok, d, t, _ = chain_case(77, B, K, V)
    ua = rng.random((B, K)).astype(np.float32) * 0.6
    U = np.concatenate([ua, rng.random((B, 2)).astype(np.float32)], axis=1)
    n, ne, toks = O.python_verify(t, d, tok, U, 0.9)
    # n = min over rows of each row's first failure of u < min(1, q/(p+1e-8))
    per_row = []
    for b in range(B):
        nb = K
        for i in range(K):
            qt = np.float32(t[b, i, tok[b, i]])
            pd = np.float32(d[b, i, tok[b, i]])
            ratio = min(np.float32(1), np.float32(qt / np.float32(pd + np.float32(1e-8))))
            if not ua[b, i] < ratio:
                nb = i
                break
        per_row.append(nb)
    assert n == min(per_row)
    np.testing.assert_array_equal(toks[:, :n], tok[:, :n])
    extra = 1 if n == K - 1 else 0
    assert ne == n + 1 + extra
    assert (toks[:, n:ne] >= 0).all() and (toks[:, ne:] == -1).all()
