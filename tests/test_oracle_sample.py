"""The sampling oracle (oracle/sample_ref.py, SwiftletSession.swift:226-273)
against what the mathematics fixes: greedy is the first maximum; the
candidates are the top-k by (logit desc, id asc) found by brute force; the
draw maps u to the token whose cumulative-probability interval holds it;
penalties only lower logits (banned ones never win).  A planted mistake
(ties to the higher id) fails."""

import numpy as np

from oracle import sample_ref as S


def _brute_topk(lg, k):
    order = sorted(range(len(lg)), key=lambda v: (-float(lg[v]), v))
    return order[:k]


def test_greedy_is_first_maximum():
    rng = np.random.default_rng(1)
    for _ in range(20):
        lg = rng.standard_normal(500).astype(np.float32)
        assert S.sample(lg, 0.0, 20, 0.8) == int(np.argmax(lg))
    lg = np.zeros(10, np.float32)
    lg[[3, 7]] = 2.0
    assert S.sample(lg, 0.0, 20, 0.8) == 3


def test_candidates_and_draw_follow_cumulative_probabilities():
    rng = np.random.default_rng(2)
    for trial in range(10):
        lg = (rng.standard_normal(3000) * 3).astype(np.float32)
        k, T = [1, 5, 20, 64][trial % 4], 0.7
        top = _brute_topk(lg, k)
        p = np.exp((lg[top].astype(np.float64) - lg[top[0]]) / T)
        cum = np.cumsum(p) / p.sum()
        # u inside each interval picks that token (top_p = 1: no cut)
        for i in range(k):
            lo = cum[i - 1] if i else 0.0
            u = (lo + cum[i]) / 2
            assert S.sample(lg, T, k, 1.0, u=u) == top[i], (trial, i)


def test_top_p_cut():
    lg = np.log(np.array([0.5, 0.3, 0.1, 0.1], np.float32))
    # T = 1: probabilities 0.5, 0.3, 0.1, 0.1; top_p 0.75 keeps the first two
    # (cumulative 0.8), 0.85 the first three
    assert S.sample(lg, 1.0, 4, 0.75, u=0.99) == 1
    assert S.sample(lg, 1.0, 4, 0.85, u=0.99) == 2
    assert S.sample(lg, 1.0, 4, 0.75, u=0.5) == 0  # 0.5 * 0.8 falls in the first interval


def test_penalties_and_banned():
    lg = np.array([1.0, 3.0, 2.9, 0.5], np.float32)
    assert S.sample(lg, 0.0, 4, 1.0) == 1
    assert S.sample(lg, 0.0, 4, 1.0, presence=0.05, frequency=0.1, seen={1: 1}) == 2  # 3 - 0.15 < 2.9
    assert S.sample(lg, 0.0, 4, 1.0, banned=[1, 2]) == 0
    for u in np.linspace(0, 0.999, 50):
        assert S.sample(lg, 0.7, 4, 1.0, banned=[1], u=u) != 1


def test_planted_mistake_is_caught():
    """Ties to the higher id in the candidate order would change the draw."""
    lg = np.array([1.0, 2.0, 2.0, 0.0], np.float32)
    want = S.sample(lg, 1.0, 2, 1.0, u=0.25)
    assert want == 1
    top_wrong = sorted(range(4), key=lambda v: (-float(lg[v]), -v))[:2]
    assert top_wrong[0] != want
