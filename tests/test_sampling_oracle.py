"""CPU tier: the sampler's oracle functions (oracle/oracle.py topk_keep,
sample_filtered, topk_greedy) against known answers derived by hand, and
against the pinned chain-path functions they reduce to."""
import numpy as np

from oracle import oracle as O


def test_topk_keep_known_answers():
    p = np.array([0.1, 0.4, 0.2, 0.2, 0.1], np.float32)
    assert O.topk_keep(p, 1).tolist() == [False, True, False, False, False]
    # the 2nd largest is 0.2, held twice: both kept
    assert O.topk_keep(p, 2).tolist() == [False, True, True, True, False]
    assert O.topk_keep(p, 3).tolist() == [False, True, True, True, False]
    assert O.topk_keep(p, 4).all() and O.topk_keep(p, 0).all() and O.topk_keep(p, 9).all()


def test_sample_filtered_known_answers():
    p = np.array([0.1, 0.4, 0.2, 0.2, 0.1], np.float32)
    # top-k 1 keeps token 1 only: every u > 0 selects it
    for u in (1e-7, 0.3, 0.999):
        assert O.sample_filtered(p, u, 1.0, 1) == 1
    # the python-mode draw takes the first prefix sum that EXCEEDS u: u = 0
    # selects the first kept token, never a filtered one (torch.multinomial
    # never returns a zero-weight index)
    assert O.sample_filtered(p, 0.0, 1.0, 1) == 1
    # past the end of the prefix sums: the last kept token
    assert O.sample_filtered(p, 1.0, 1.0, 1) == 1
    assert O.sample_filtered(p, 1.0, 1.0, 2) == 3
    # top-k 2 keeps {1, 2, 3} with mass 0.8: normalised 0.5, 0.25, 0.25
    assert O.sample_filtered(p, 0.49, 1.0, 2) == 1
    assert O.sample_filtered(p, 0.51, 1.0, 2) == 2
    assert O.sample_filtered(p, 0.8, 1.0, 2) == 3
    # no filter: the plain sequential inverse CDF over p / sum(p)
    rng = np.random.default_rng(0)
    q = rng.random(50).astype(np.float32)
    q /= q.sum()
    for u in rng.random(20):
        assert O.sample_filtered(q, u, 1.0, 0) == O.sample_weights(q, u)


def test_sample_filtered_top_p_matches_python_verify_bonus():
    """With K = 0 the python-mode verification is one filtered bonus draw."""
    rng = np.random.default_rng(1)
    for top_p in (0.3, 0.9):
        p = rng.dirichlet(np.ones(64)).astype(np.float32)[None, None, :]
        for u in rng.random(10).astype(np.float32):
            _, ne, toks = O.python_verify(p, np.zeros((1, 0, 64), np.float32),
                                          np.zeros((1, 0), np.int32),
                                          np.array([[u, 0.5]], np.float32), top_p)
            assert ne == 1
            assert O.sample_filtered(p[0, 0], u, top_p, 0) == toks[0, 0]


def test_topk_greedy_known_answers():
    x = np.array([[1.0, 3.0, 3.0, 2.0, -1.0],
                  [0.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    assert O.topk_greedy(x, 1).tolist() == [[1], [0]]
    assert O.topk_greedy(x, 3).tolist() == [[1, 2, 3], [0, 1, 2]]
    assert O.topk_greedy(x[:1], 5).tolist() == [[1, 2, 3, 0, 4]]
    # k = 1 is the first argmax
    rng = np.random.default_rng(2)
    y = rng.integers(0, 4, (20, 30)).astype(np.float32)
    assert O.topk_greedy(y, 1)[:, 0].tolist() == [O.argmax_first(r) for r in y]
