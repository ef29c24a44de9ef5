"""GPU parity: the sampler's candidate distribution on the device.

Reference: the final distribution of Sampler._transformed (serve/sampler.py:85-112:
top_k -> drop -inf -> softmax -> top_p -> min_p -> softmax(v / T)), checked
against the oracle's restatement (oracle.cpp or_sample_dist, pinned in
tests/test_oracle_sampler.py) fed by the oracle's vocab pass. Gate: candidate
ids and counts identical, probabilities within 2e-6 absolute (the device takes
f32 exponentials of exactly formed differences and f64 sums; the reference's
numpy float32 sums pin no bits). Every row's top_p cut and min_p ratios lie at
least 1e-5 away from the thresholds, so the f32 / f64 difference cannot move
a cut; the test asserts that of its inputs.
"""
import numpy as np
import pytest
from scipy.special import softmax

import oracle as O
from util import F32, to_dev

pytestmark = pytest.mark.gpu

MARGIN = 1e-5


def assert_away_from_cuts(tv, top_p, min_p):
    """the inputs' cumulative shares and ratios are not near top_p / min_p"""
    for r in range(tv.shape[0]):
        v = tv[r][np.isfinite(tv[r])]
        if v.size == 0:
            continue
        p = softmax(v)
        if top_p < 1.0:
            assert np.min(np.abs(np.cumsum(p) - np.float32(top_p))) > MARGIN, r
        if min_p > 0.0:
            assert np.min(np.abs(p / p[0] - np.float32(min_p))) > MARGIN, r


def check_rows(ids, probs, n, L, K, temp, top_p, min_p):
    _, oam, oti, otv = O.vocab_reduce(L, K)
    assert_away_from_cuts(otv, top_p, min_p)
    rid, rp, rn = O.sample_dist(oti, otv, oam, temp, top_p, min_p)
    for r in range(L.shape[0]):
        assert n[r] == rn[r], (r, n[r], rn[r])
        assert np.array_equal(ids[r, :n[r]], rid[r, :rn[r]]), r
        assert np.abs(probs[r, :n[r]].astype(np.float64) - rp[r, :rn[r]]).max() <= 2e-6, r
        assert abs(float(probs[r, :n[r]].astype(np.float64).sum()) - 1.0) <= 1e-5


@pytest.mark.parametrize("top_k,top_p,min_p,temp", ((64, 0.95, 0.0, 0.7), (64, 1.0, 0.0, 1.0), (40, 0.9, 0.05, 0.8),
                                                    (256, 0.5, 0.0, 1.3), (1, 0.95, 0.0, 0.7), (64, 0.95, 0.0, 0.0)))
def test_dist_matches_oracle(prims, top_k, top_p, min_p, temp):
    rows, V = 12, 30000
    L = O.to_f64(O.normal(41, (rows, V), 0.0, 2.0, F32), F32)
    L[3, :] = -np.inf                   # fully masked row: point mass on the argmax
    L[4, 10:] = -np.inf                 # fewer finite logits than top_k
    L[5, :] *= 4.0                      # a peaked row
    dL = to_dev(O.from_f64(L, F32), F32)
    lse, am, ti, tv = prims.vocab_reduce(dL, top_k)
    ids, probs, n = prims.sample_dist(ti, tv, am, temp, top_p, min_p)
    check_rows(ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy(), L, top_k, temp, top_p, min_p)


def test_tail_then_dist(prims):
    """output tail fused into the vocab pass, then the distribution: the oracle's
    softcap (pinned bitwise to apply_output_tail) followed by its sampler"""
    rows, V = 4, 50000
    L = O.to_f64(O.normal(42, (rows, V), 0.0, 8.0, F32), F32)
    Z = O.softcap(L, 1.0, 30.0, F32)
    dL = to_dev(O.from_f64(L, F32), F32)
    lse, am, ti, tv = prims.vocab_reduce_tail(dL, 1.0, 30.0, 64)
    ids, probs, n = prims.sample_dist(ti, tv, am, 0.7, 0.95, 0.0)
    check_rows(ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy(), Z, 64, 0.7, 0.95, 0.0)
