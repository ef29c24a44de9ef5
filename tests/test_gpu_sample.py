"""GPU parity: the sampler's candidate distribution on the device.

Reference: serve/sampler.py:43-112 (Sampler._transformed: top_k -> drop -inf ->
softmax -> top_p -> min_p -> softmax(x / temperature)), restated below in the
same numpy float32 steps. The reference's probabilities come from numpy's own
float32 exp and pairwise sums, which nothing pins bitwise; the device values
must match them within 2e-6 absolute, and the candidate ids and counts exactly
(inputs are drawn without near-ties at the top_p / min_p cuts).
"""
import numpy as np
import pytest

import oracle as O
from util import F32, to_dev

pytestmark = pytest.mark.gpu


def ref_dist(lg, top_k, top_p, min_p, temperature):
    lg = lg.astype(np.float32)
    if not np.isfinite(lg).any() or temperature <= 0:
        return np.array([int(np.argmax(lg))]), np.array([1.0], np.float32)
    k = min(top_k, lg.size)
    cand = np.argpartition(-lg, k - 1)[:k]
    cl = lg[cand]
    order = np.argsort(-cl, kind="stable")
    cand, cl = cand[order], cl[order]
    keep = cl > -np.inf
    cand, cl = cand[keep], cl[keep]
    if cand.size == 0:
        return np.array([int(np.argmax(lg))]), np.array([1.0], np.float32)

    def softmax(x):
        e = np.exp(x - x.max())
        return e / e.sum()

    probs = softmax(cl)
    if top_p < 1.0:
        n = int(np.searchsorted(np.cumsum(probs), top_p) + 1)
        cand, cl, probs = cand[:n], cl[:n], probs[:n]
    if min_p > 0.0:
        keep = probs >= min_p * probs.max()
        cand, cl = cand[keep], cl[keep]
    final = softmax(cl / np.float32(temperature))
    return cand, final / final.sum()


@pytest.mark.parametrize("top_k,top_p,min_p,temp", ((64, 0.95, 0.0, 0.7), (64, 1.0, 0.0, 1.0), (40, 0.9, 0.05, 0.8),
                                                    (256, 0.5, 0.0, 1.3), (1, 0.95, 0.0, 0.7), (64, 0.95, 0.0, 0.0)))
def test_dist_matches_reference(prims, top_k, top_p, min_p, temp):
    rows, V = 12, 30000
    L = O.to_f64(O.normal(41, (rows, V), 0.0, 2.0, F32), F32)
    L[3, :] = -np.inf                   # fully masked row: point mass on the argmax
    L[4, 10:] = -np.inf                 # fewer finite logits than top_k
    L[5, :] *= 4.0                      # a peaked row
    dL = to_dev(O.from_f64(L, F32), F32)
    lse, am, ti, tv = prims.vocab_reduce(dL, top_k)
    ids, probs, n = prims.sample_dist(ti, tv, am, temp, top_p, min_p)
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        rc, rp = ref_dist(L[r], top_k, top_p, min_p, temp)
        assert n[r] == rc.size, (r, n[r], rc.size)
        assert np.array_equal(ids[r, :n[r]], rc), r
        assert np.abs(probs[r, :n[r]] - rp).max() <= 2e-6, r
        assert abs(float(probs[r, :n[r]].astype(np.float64).sum()) - 1.0) <= 1e-5


def test_tail_then_dist(prims):
    """output tail fused into the vocab pass, then the distribution: the same as
    softcap followed by the reference sampler"""
    rows, V = 4, 50000
    L = O.to_f64(O.normal(42, (rows, V), 0.0, 8.0, F32), F32)
    Z = O.softcap(L, 1.0, 30.0, F32)
    dL = to_dev(O.from_f64(L, F32), F32)
    lse, am, ti, tv = prims.vocab_reduce_tail(dL, 1.0, 30.0, 64)
    ids, probs, n = prims.sample_dist(ti, tv, am, 0.7, 0.95, 0.0)
    for r in range(rows):
        rc, rp = ref_dist(Z[r], 64, 0.95, 0.0, 0.7)
        assert n[r].item() == rc.size and np.array_equal(ids[r, :rc.size].cpu().numpy(), rc)
        assert np.abs(probs[r, :rc.size].cpu().numpy() - rp).max() <= 2e-6
