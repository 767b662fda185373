"""Pins of the oracle's sampler (or_philox4x32_10, or_sample), independent of its code:
Philox4x32-10's published known-answer vectors (Random123's kat_vectors), the greedy
special cases (temperature 0, top_k 1, a vanishing top_p, the argmax tie rule with -0 == +0),
the candidate set against a numpy ranking, and the empirical distribution of many draws
against the float64 softmax-with-cuts probabilities (chi-square)."""
import numpy as np
import pytest
from scipy import stats

from oracle import oracle


@pytest.mark.parametrize("ctr,key,exp", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, exp):
    assert oracle.philox4x32_10(ctr, key) == exp


def test_greedy_special_cases():
    rng = np.random.default_rng(1)
    l = rng.standard_normal(1000).astype(np.float32)
    l[[17, 400, 901]] = 9.0          # a three-way tie for the maximum: index 17 wins
    for c in range(20):
        assert oracle.sample(l, 0.0, 40, 0.9, 5, c) == 17
        assert oracle.sample(l, -1.0, 40, 0.9, 5, c) == 17
        assert oracle.sample(l, 1.0, 1, 1.0, 5, c) == 17
        assert oracle.sample(l, 1.0, 50, 1e-9, 5, c) == 17
    z = np.array([-1.0, -0.0, 0.0, -2.0], np.float32)   # -0 at index 1 ties +0 at index 2
    assert oracle.sample(z, 0.0, 10, 1.0, 0, 0) == 1
    z2 = np.array([-1.0, 0.0, -0.0], np.float32)
    assert oracle.sample(z2, 0.0, 10, 1.0, 0, 0) == 1


def test_non_finite_weights_draw_the_argmax():
    """A temperature so small that 1/T overflows, and a +inf top logit, would make every weight
    exp(0 * inf) or exp(inf - inf) = NaN: both draw greedily (the argmax, lowest index)."""
    rng = np.random.default_rng(4)
    l = rng.standard_normal(5000).astype(np.float32)
    l[[33, 700]] = 7.5
    assert np.isinf(np.float32(1.0) / np.float32(1e-39))
    for c in range(10):
        assert oracle.sample(l, 1e-39, 40, 0.9, 3, c) == 33
        assert oracle.sample(l, np.float32(2.0e-39), 1024, 1.0, 3, c) == 33
    li = l.copy()
    li[[91, 4000]] = np.inf
    for c in range(10):
        assert oracle.sample(li, 0.8, 40, 0.95, 3, c) == 91


def test_candidates_are_the_ranked_top_k():
    rng = np.random.default_rng(2)
    l = np.round(rng.standard_normal(3000), 1).astype(np.float32)   # many ties
    k = 37
    order = np.lexsort((np.arange(l.size), -l.astype(np.float64)))
    top = set(order[:k].tolist())
    seen = set()
    for c in range(4000):
        t = oracle.sample(l, 1e30, k, 1.0, 11, c)      # huge T: every candidate weighs ~1
        assert t in top
        seen.add(t)
    assert seen == top


def _probs(l, T, k, p):
    order = np.lexsort((np.arange(l.size), -l.astype(np.float64)))[:k]
    w = np.exp((l[order].astype(np.float64) - float(l[order[0]])) / T)
    c = np.cumsum(w)
    n = int(np.argmax(c >= p * c[-1])) + 1 if p < 1 else k
    return order[:n], w[:n] / c[n - 1]


@pytest.mark.parametrize("T,k,p", [(0.8, 6, 1.0), (1.3, 40, 0.9), (0.5, 1024, 0.95)])
def test_draws_follow_the_distribution(T, k, p):
    rng = np.random.default_rng(3)
    l = (rng.standard_normal(50) * 1.5).astype(np.float32)
    ids, pr = _probs(l, T, k, p)
    N = 30000
    draws = np.array([oracle.sample(l, T, k, p, 99, c) for c in range(N)])
    assert set(np.unique(draws).tolist()) <= set(ids.tolist())
    obs = np.array([(draws == i).sum() for i in ids], np.float64)
    keep = pr * N >= 5                       # chi-square cells with enough expectation
    exp = pr[keep] * N
    o = obs[keep]
    rest_o, rest_e = N - o.sum(), N - exp.sum()
    if rest_e >= 5:
        o, exp = np.append(o, rest_o), np.append(exp, rest_e)
    chi2 = ((o - exp) ** 2 / exp).sum()
    assert stats.chi2.sf(chi2, len(o) - 1) > 1e-4, (chi2, len(o))


def test_counter_and_seed_streams_differ():
    l = np.zeros(64, np.float32)
    a = [oracle.sample(l, 1.0, 64, 1.0, 1, c) for c in range(200)]
    b = [oracle.sample(l, 1.0, 64, 1.0, 2, c) for c in range(200)]
    assert a != b and len(set(a)) > 40
