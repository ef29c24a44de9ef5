"""CPU: the oracle's sampler distribution (oracle.cpp or_sample_dist, the final
candidate distribution of Sampler._transformed, serve/sampler.py:85-112),
pinned by what the definition fixes rather than by a second copy of its steps:

  * top_p = 1, min_p = 0: the distribution is softmax(v / T) over the finite
    candidates (scipy.special.softmax on the f32 quotients);
  * the top_p cut is the shortest prefix whose cumulative probability reaches
    top_p, brute-forced with exact fractions on rows whose probabilities are
    known exactly (v = log w) and whose cut lies well away from top_p;
  * the min_p rule keeps p_i >= min_p * p_max, brute-forced the same way;
  * temperature <= 0, and rows with no finite candidate, give the point mass
    on the argmax; -inf candidates never enter;
  * the probabilities sum to 1 and their ratios are exp((v_i - v_j) / T).
"""
from fractions import Fraction

import numpy as np
import pytest
from scipy.special import softmax

import oracle as O

RNG = np.random.default_rng(2026)


def f32q(v, T):
    """v / T as numpy's float32 division gives it (sampler.py:111)"""
    return (np.asarray(v, np.float32) / np.float32(T)).astype(np.float64)


def row_from_weights(w, K):
    """a sorted candidate row whose softmax is w / sum(w) (v = log w, descending),
    padded with -inf to K"""
    w = sorted(w, reverse=True)
    v = np.full(K, -np.inf)
    v[:len(w)] = np.log(np.asarray(w, np.float64))
    return v


def run(vals, T, top_p, min_p, ids=None, amax=None):
    vals = np.atleast_2d(vals)
    rows, K = vals.shape
    if ids is None:
        ids = np.tile(np.arange(K, dtype=np.int64) * 7 + 3, (rows, 1))
    if amax is None:
        amax = ids[:, 0].copy()
    return O.sample_dist(ids, vals, amax, T, top_p, min_p)


@pytest.mark.parametrize("T", (1.0, 0.7, 1.3, 0.05))
def test_no_filters_is_softmax_over_v_by_t(T):
    K = 64
    vals = np.sort(RNG.normal(0, 3, (8, K)), axis=1)[:, ::-1].copy()
    vals[2, 50:] = -np.inf
    vals = vals.astype(np.float32).astype(np.float64)  # logits are f32 values
    ids, p, n = run(vals, T, 1.0, 0.0)
    for r in range(8):
        fin = np.isfinite(vals[r])
        assert n[r] == fin.sum()
        want = softmax(f32q(vals[r, fin], T))
        assert np.allclose(p[r, :n[r]], want, rtol=1e-14, atol=0)
        assert np.array_equal(ids[r, :n[r]], (np.arange(K) * 7 + 3)[fin])
        assert abs(p[r, :n[r]].sum() - 1.0) < 1e-14


def brute_cut(w, top_p):
    """shortest prefix of w (descending) whose exact cumulative share reaches top_p"""
    W = sum(Fraction(x) for x in w)
    run_ = Fraction(0)
    tp = Fraction(float(np.float32(top_p)))
    for k, x in enumerate(w, 1):
        run_ += Fraction(x) / W
        if run_ >= tp:
            return k
    return len(w)


def test_top_p_cut_brute_force():
    checked = 0
    for _ in range(300):
        m = int(RNG.integers(1, 40))
        w = sorted((int(x) for x in RNG.integers(1, 1000, m)), reverse=True)
        W = sum(w)
        cums = np.cumsum(w) / W
        # top_p at least 1e-3 away from every cumulative share
        top_p = float(RNG.uniform(0.05, 0.99))
        if np.min(np.abs(cums - top_p)) < 1e-3:
            continue
        _, p, n = run(row_from_weights(w, 64), 1.0, top_p, 0.0)
        k = brute_cut(w, top_p)
        assert n[0] == k, (w, top_p, n[0], k)
        # the kept candidates renormalize among themselves (T = 1: p_i = w_i / sum of the kept,
        # up to the f32 rounding of v / T: |v| < 7 moves p by < 1e-6 relative)
        assert np.allclose(p[0, :k], np.asarray(w[:k], np.float64) / sum(w[:k]), rtol=1e-6, atol=0)
        checked += 1
    assert checked > 150


def test_top_p_at_or_above_the_total_keeps_all():
    w = [5, 3, 2, 1]
    _, _, n = run(row_from_weights(w, 8), 1.0, 0.9999999, 0.0)
    assert n[0] == 4
    _, _, n = run(row_from_weights(w, 8), 1.0, 1.0, 0.0)
    assert n[0] == 4


def test_min_p_brute_force():
    checked = 0
    for _ in range(300):
        m = int(RNG.integers(1, 40))
        w = sorted((int(x) for x in RNG.integers(1, 1000, m)), reverse=True)
        ratios = np.asarray(w, np.float64) / w[0]
        min_p = float(RNG.uniform(0.01, 1.0))
        if np.min(np.abs(ratios - min_p)) < 1e-3:
            continue
        ids, p, n = run(row_from_weights(w, 64), 1.0, 1.0, min_p)
        mp = Fraction(float(np.float32(min_p)))
        keep = [i for i, x in enumerate(w) if Fraction(x) >= mp * Fraction(w[0])]
        assert n[0] == len(keep)
        assert np.array_equal(ids[0, :n[0]], (np.arange(64) * 7 + 3)[keep])
        kw = np.asarray([w[i] for i in keep], np.float64)
        assert np.allclose(p[0, :n[0]], kw / kw.sum(), rtol=1e-6, atol=0)
        checked += 1
    assert checked > 150


def test_top_p_then_min_p_order():
    """min_p applies to the candidates the top_p cut kept (sampler.py:104-109)"""
    w = [40, 30, 20, 6, 4]  # shares .4 .3 .2 .06 .04
    _, _, n = run(row_from_weights(w, 8), 1.0, 0.85, 0.0)
    assert n[0] == 3  # .4 + .3 = .7 < .85 <= .9
    _, _, n = run(row_from_weights(w, 8), 1.0, 0.85, 0.6)
    assert n[0] == 2  # of the three, 30 >= .6 * 40 and 20 < 24


@pytest.mark.parametrize("T", (0.0, -1.0))
def test_greedy_is_point_mass_on_argmax(T):
    vals = np.sort(RNG.normal(0, 1, (2, 16)), axis=1)[:, ::-1].copy()
    ids, p, n = run(vals, T, 0.9, 0.1, amax=np.array([123, 456], np.int64))
    assert list(n) == [1, 1] and list(ids[:, 0]) == [123, 456] and list(p[:, 0]) == [1.0, 1.0]


def test_all_masked_row_is_point_mass_on_argmax():
    vals = np.full((1, 16), -np.inf)
    ids, p, n = run(vals, 0.8, 0.9, 0.0, amax=np.array([77], np.int64))
    assert n[0] == 1 and ids[0, 0] == 77 and p[0, 0] == 1.0


def test_ratios_follow_temperature():
    vals = np.sort(RNG.normal(0, 2, (1, 32)), axis=1)[:, ::-1].astype(np.float32).astype(np.float64)
    T = 0.6
    _, p, n = run(vals, T, 0.95, 0.02)
    q = f32q(vals[0, :n[0]], T)
    assert np.allclose(p[0, 1:n[0]] / p[0, 0], np.exp(q[1:] - q[0]), rtol=1e-13)
    assert abs(p[0, :n[0]].sum() - 1.0) < 1e-14


def test_plausible_mistakes_are_caught():
    """equality cases the checks above cannot build from random weights: an
    off-by-one cut, a strict min_p comparison or a temperature applied before
    the top_p softmax would each fail here"""
    half = np.log(0.5)  # exp(log 0.5) is exactly 0.5, so the T = 1 shares are .5, .25, .25 exactly
    row = np.array([[0.0, half, half, -np.inf]])
    _, p, n = run(row, 1.0, 1.0, 0.0)
    assert n[0] == 3 and np.allclose(p[0, :3], [0.5, 0.25, 0.25], rtol=1e-6, atol=0)
    _, _, n = run(row, 1.0, 0.75, 0.0)
    assert n[0] == 2  # .5 + .25 reaches .75 exactly: searchsorted's left side, plus one
    _, _, n = run(row, 1.0, 1.0, 0.5)
    assert n[0] == 3  # .25 >= .5 * .5 with equality: ">=" keeps it
    # at T = 0.25 the final distribution sharpens, but the top_p cut uses the T = 1 shares
    _, _, n = run(row_from_weights([60, 30, 10], 4), 0.25, 0.8, 0.0)
    assert n[0] == 2


# ---------------------------------------------------------------- full rows
# oracle.sample_rows (any top_k, on full rows of edited logits) against the
# reference's own Sampler._transformed: tests/golden/sampler.npz, written by
# tests/golden/make_sampler_golden.py from serve/sampler.py. The golden rows
# include the cuts no closed form fixes (top_p equal to one of the row's
# float32 cumulative sums and the next float above it, min_p at a probability
# ratio), the fully masked fallback under a bias, greedy after a bias, top_k
# above 256 and above V, top_k <= 0 with and without top_p.
GOLD_SAMPLER = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                                  "sampler.npz"))


def gold_rows():
    return range(GOLD_SAMPLER["raw"].shape[0])


@pytest.mark.parametrize("r", gold_rows())
def test_sample_rows_matches_reference_golden(r):
    g = GOLD_SAMPLER
    T, k, tp, mp = g["params"][r]
    (ids, probs), = O.sample_rows(g["edited"][r:r + 1], g["raw_argmax"][r:r + 1], int(k), T, tp, mp)
    n = int(g["count"][r])
    assert len(ids) == n
    assert np.array_equal(ids, g["cand"][r, :n])
    # the same float32 operations in the same order: the same bits
    assert np.array_equal(probs, g["probs"][r, :n])


def test_sample_rows_golden_covers_the_edges():
    g = GOLD_SAMPLER
    kinds = set(g["kind"].tolist())
    assert kinds == {0, 1, 2}                       # dist, greedy, masked
    masked = np.nonzero(g["kind"] == 2)[0]
    assert all(g["cand"][r, 0] == g["raw_argmax"][r] for r in masked)
    # an edited argmax that differs from the raw one (bias, mask, penalties)
    moved = [r for r in gold_rows() if np.isfinite(g["edited"][r]).any()
             and np.argmax(g["edited"][r]) != g["raw_argmax"][r]]
    assert moved
    assert (g["params"][:, 1] <= 0).any() and (g["params"][:, 1] > 256).any()
    assert g["boundary"].sum() >= 6
    # the nudged top_p rows cut one candidate later than the exact ones
    b = np.nonzero(g["boundary"])[0]
    assert any(g["count"][i + 1] == g["count"][i] + 1 for i in b[:-1])


def test_sample_rows_planted_strict_cut_fails():
    """a top_p cut taken with '>' instead of '>=' misses the boundary rows"""
    g = GOLD_SAMPLER
    hit = 0
    for r in np.nonzero(g["boundary"])[0]:
        T, k, tp, mp = g["params"][r]
        if mp > 0:
            continue
        x = g["edited"][r].astype(np.float32)
        srt = np.sort(x)[::-1]
        e = np.exp(srt - srt.max())
        cs = np.cumsum(e / e.sum())
        wrong = int(np.searchsorted(cs, tp, side="right")) + 1
        hit += wrong != g["count"][r]
    assert hit >= 1
