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
GOLD_SAMPLER = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                                  "sampler.npz"))

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


# ------------------------------------------------------- the masked fallback
def test_masked_fallback_takes_the_raw_argmax(prims):
    """serve/sampler.py:70-74: with no finite edited logit the point mass goes to
    np.argmax of the RAW logits, not of the edited ones. Golden rows from the
    reference (a full mask, and a full mask over a bias that moved the argmax),
    run through the vocab pass on the edited rows and mg_sample_dist with the
    raw rows' argmax; a row whose mask leaves tokens keeps its distribution."""
    import torch
    g = GOLD_SAMPLER
    rows = [r for r in range(g["raw"].shape[0]) if g["kind"][r] == 2]
    rows.append(int(np.nonzero((g["params"][:, 1] == 64) & (g["kind"] == 0))[0][0]))
    raw = torch.from_numpy(g["raw"][rows]).cuda()
    ed = torch.from_numpy(g["edited"][rows]).cuda()
    _, ram, _, _ = prims.vocab_reduce(raw, 64)
    _, am, ti, tv = prims.vocab_reduce(ed, 64)
    ids, probs, n = prims.sample_dist(ti, tv, am, 0.7, 0.95, 0.0, raw_argmax=ram)
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for i, r in enumerate(rows):
        c = int(g["count"][r])
        assert n[i] == c
        assert np.array_equal(ids[i, :c], g["cand"][r, :c]), r
        assert np.abs(probs[i, :c].astype(np.float64) - g["probs"][r, :c]).max() <= 2e-6
    # the masked rows' raw argmax differs from what the edited rows give
    assert any(int(am[i]) != int(g["raw_argmax"][r]) for i, r in enumerate(rows[:-1]))


# ---------------------------------------------------------- any top_k, full rows


def test_sample_rows_matches_reference_golden(prims):
    """mg_sample_rows on the reference's own edited rows (top_k 64, 0, -1, 300,
    1000, 5000 > V; index-order outputs; bias, penalties, masks; greedy; masked;
    -inf entries): identical ids and counts, probabilities within 2e-6. Rows
    marked `boundary` put top_p exactly on one of the row's float32 cumulative
    sums (or the next float): the device sums exp in f64, the reference in
    float32, so there the cut may fall one candidate apart; the ids the two
    share must agree and the device's cut must lie within 1e-6 of top_p."""
    import torch
    g = GOLD_SAMPLER
    rows = g["raw"].shape[0]
    for r in range(rows):
        T, k, tp, mp = g["params"][r]
        ed = torch.from_numpy(g["edited"][r:r + 1]).cuda()
        ram = torch.from_numpy(g["raw_argmax"][r:r + 1]).cuda()
        ids, probs, n = prims.sample_rows(ed, int(k), T, tp, mp, raw_argmax=ram)
        n = int(n.cpu()[0])
        ids = ids.cpu().numpy()[0, :n]
        probs = probs.cpu().numpy()[0, :n].astype(np.float64)
        c = int(g["count"][r])
        if g["boundary"][r] and n != c:
            assert abs(n - c) == 1, (r, n, c)
            m = min(n, c)
            assert np.array_equal(ids[:m], g["cand"][r, :m]), r
            x = g["edited"][r].astype(np.float64)
            e = np.exp(np.sort(x)[::-1] - x.max())
            cs = np.cumsum(e / e.sum())
            assert abs(cs[m - 1] - np.float32(tp)) <= 1e-6, (r, cs[m - 1], tp)
            continue
        assert n == c, (r, n, c)
        assert np.array_equal(ids, g["cand"][r, :c]), r
        assert np.abs(probs - g["probs"][r, :c]).max() <= 2e-6, r
        assert abs(probs.sum() - 1.0) <= 1e-5


@pytest.mark.parametrize("top_k,top_p,min_p,temp", ((0, 0.95, 0.0, 1.0), (0, 0.95, 0.02, 0.7), (0, 1.0, 0.01, 1.0),
                                                    (1000, 1.0, 0.0, 0.8), (3000, 0.95, 0.0, 1.0),
                                                    (10000, 0.95, 0.0, 1.0)))
def test_sample_rows_vocab_scale(prims, top_k, top_p, min_p, temp):
    """[8, 201088] rows at the vocab pass's shape against oracle.sample_rows (pinned
    to the reference above): top_k = 0 with top_p = 0.95 (nuclei of a few hundred
    to a few thousand tokens), index-order outputs, top_k far above 256. Rows built
    with their cuts away from top_p / min_p (asserted), so both precisions agree."""
    import torch
    rows, V = 8, 201088
    L = O.from_f64(O.to_f64(O.normal(51, (rows, V), 0.0, 1.0, F32), F32), F32).view(np.float32).copy()
    # scales 3..7: 0.95-nuclei from about 18 000 tokens (beyond the device's sort) down to 6
    L *= np.array([3.0, 3.5, 4.0, 4.5, 5.0, 5.5, 6.0, 7.0], np.float32)[:, None]
    L[2, ::3] = -np.inf
    for r in range(rows):
        x = np.sort(L[r][np.isfinite(L[r])])[::-1]
        kk = top_k if 0 < top_k < x.size else x.size
        p64 = softmax(x[:kk].astype(np.float64))
        e32 = np.exp(x[:kk] - x[0])
        p32 = e32 / e32.sum()
        if top_p < 1.0:
            # the float32 and the exact cumulative sums cut at the same place, or
            # both beyond what the device sorts (numpy's float32 cumsum drifts by
            # up to ~1e-5 over tens of thousands of terms and moves long cuts)
            c32 = np.searchsorted(np.cumsum(p32), np.float32(top_p)) + 1
            c64 = np.searchsorted(np.cumsum(p64), np.float64(np.float32(top_p))) + 1
            assert c32 == c64 or min(c32, c64) > 4096, (r, c32, c64)
        if min_p > 0.0:
            assert np.min(np.abs(p64 / p64[0] - np.float32(min_p))) > 1e-6, r
    want = O.sample_rows(L, np.argmax(L, axis=1), top_k, temp, top_p, min_p)
    ids, probs, n = prims.sample_rows(torch.from_numpy(L).cuda(), top_k, temp, top_p, min_p)
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        wi, wp = want[r]
        if len(wi) > 4096 and (top_k > 0 or top_p < 1.0):
            assert n[r] == -1, r                  # more sorted candidates than the device sorts
            continue
        assert n[r] == len(wi), (r, n[r], len(wi))
        assert np.array_equal(ids[r, :n[r]], wi), r
        assert np.abs(probs[r, :n[r]].astype(np.float64) - wp).max() <= 2e-6, r


@pytest.mark.parametrize("tied", (False, True))
def test_sample_rows_crowded_threshold_bin(prims, tied):
    """the 4096th largest candidate in a bin of the 12-bit image prefix that holds
    60 000 candidates (all of them in [1, 1.1), or all equal to 1.0): more than
    the gathering room, so the rows take the radix selection (ties broken by
    index) and the ordered compaction; 3000 larger logits hold the nucleus"""
    import torch
    rows, V = 2, 201088
    rng = np.random.default_rng(52)
    L = np.full((rows, V), -5.0, np.float32)
    for r in range(rows):
        pos = rng.permutation(V)
        L[r, pos[:3000]] = rng.uniform(10.0, 12.0, 3000).astype(np.float32)
        L[r, pos[3000:63000]] = 1.0 if tied else rng.uniform(1.0, 1.1, 60000).astype(np.float32)
    for top_k, top_p in ((0, 0.95), (20000, 0.9)):
        for r in range(rows):
            # the float32 and exact cumulative sums cut at the same place
            x = np.sort(L[r])[::-1][:top_k or V]
            e32 = np.exp(x - x[0])
            p64 = softmax(x.astype(np.float64))
            c32 = np.searchsorted(np.cumsum(e32 / e32.sum()), np.float32(top_p)) + 1
            c64 = np.searchsorted(np.cumsum(p64), np.float64(np.float32(top_p))) + 1
            assert c32 == c64 and c32 < 3000, (r, c32, c64)
        want = O.sample_rows(L, np.argmax(L, axis=1), top_k, 1.0, top_p, 0.0)
        ids, probs, n = prims.sample_rows(torch.from_numpy(L).cuda(), top_k, 1.0, top_p, 0.0)
        ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
        for r in range(rows):
            wi, wp = want[r]
            assert n[r] == len(wi), (top_k, r, n[r], len(wi))
            assert np.array_equal(ids[r, :n[r]], wi), (top_k, r)
            assert np.abs(probs[r, :n[r]].astype(np.float64) - wp).max() <= 2e-6, (top_k, r)


def test_sample_rows_threshold_bin_on_top(prims):
    """the 4096 largest candidates all in the top bin of the image prefix (992 <=
    x < 1024, a bin 32 wide), nothing above it: the whole sorted prefix comes
    from the gathered threshold bin"""
    import torch
    V = 20000
    rng = np.random.default_rng(53)
    L = np.full((1, V), -5.0, np.float32)
    L[0, rng.permutation(V)[:4096]] = rng.uniform(992.0, 1024.0, 4096).astype(np.float32)
    want = O.sample_rows(L, np.argmax(L, axis=1), 0, 8.0, 0.95, 0.0)
    ids, probs, n = prims.sample_rows(torch.from_numpy(L).cuda(), 0, 8.0, 0.95, 0.0)
    (wi, wp), = want
    assert int(n.cpu()[0]) == len(wi)
    assert np.array_equal(ids.cpu().numpy()[0, :len(wi)], wi)
    assert np.abs(probs.cpu().numpy()[0, :len(wi)].astype(np.float64) - wp).max() <= 2e-6


@pytest.mark.parametrize("temp", (1.0, 0.0))
def test_sample_rows_split_rows(prims, temp):
    """rows of V >= 16384 with sorted outputs and no top_k cut run split over
    several work-groups per row: a fully masked row (the raw argmax), NaN and
    -inf entries, a row whose maximum sits in the last slice, and greedy rows
    (temperature 0: np.argmax, NaN counting as the largest) beside sampled ones"""
    import torch
    rows, V = 5, 30000
    L = O.normal(57, (rows, V), 0.0, 3.0, F32).view(np.float32).copy()
    L[0] = -np.inf
    L[1, ::7] = np.nan
    L[2, ::3] = -np.inf
    L[3, V - 1] = 40.0
    L[4, 12345] = np.nan
    raw = np.array([17, 0, 0, 0, 0], np.int64)
    for r in range(rows):
        f = np.isfinite(L[r])
        if f.any():
            x = np.sort(L[r][f])[::-1]
            e32 = np.exp(x - x[0])
            p64 = softmax(x.astype(np.float64))
            c32 = np.searchsorted(np.cumsum(e32 / e32.sum()), np.float32(0.9)) + 1
            c64 = np.searchsorted(np.cumsum(p64), np.float64(np.float32(0.9))) + 1
            assert c32 == c64, (r, c32, c64)
    want = O.sample_rows(L, raw, 0, temp, 0.9, 0.0)
    ids, probs, n = prims.sample_rows(torch.from_numpy(L).cuda(), 0, temp, 0.9, 0.0,
                                      raw_argmax=torch.from_numpy(raw).cuda())
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        wi, wp = want[r]
        assert n[r] == len(wi), (r, n[r], len(wi))
        assert np.array_equal(ids[r, :n[r]], wi), r
        assert np.abs(probs[r, :n[r]].astype(np.float64) - wp).max() <= 2e-6, r


@pytest.mark.parametrize("V,ld", ((30001, 30001), (40000, 40003), (50000, 50000)))
def test_sample_rows_split_unaligned(prims, V, ld):
    """the split path on rows whose slices start off 16-byte boundaries (odd V or
    row stride: entry-by-entry loads there), and on aligned rows of three rows"""
    import torch
    rows = 3
    wide = O.normal(58, (rows, ld), 0.0, 3.0, F32).view(np.float32).copy()
    L = wide[:, :V]
    for r in range(rows):
        x = np.sort(L[r])[::-1]
        e32 = np.exp(x - x[0])
        p64 = softmax(x.astype(np.float64))
        c32 = np.searchsorted(np.cumsum(e32 / e32.sum()), np.float32(0.9)) + 1
        c64 = np.searchsorted(np.cumsum(p64), np.float64(np.float32(0.9))) + 1
        assert c32 == c64, (r, c32, c64)
    want = O.sample_rows(np.ascontiguousarray(L), np.argmax(L, axis=1), 0, 1.0, 0.9, 0.0)
    ids, probs, n = prims.sample_rows(torch.from_numpy(wide).cuda()[:, :V], 0, 1.0, 0.9, 0.0)
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        wi, wp = want[r]
        assert n[r] == len(wi), (r, n[r], len(wi))
        assert np.array_equal(ids[r, :n[r]], wi), r
        assert np.abs(probs[r, :n[r]].astype(np.float64) - wp).max() <= 2e-6, r


@pytest.mark.parametrize("rows", (64, 100))
def test_sample_rows_split_fewer_slices(prims, rows):
    """64 rows split over 4 work-groups each (the bench's shape at a smaller V),
    100 rows over 2"""
    import torch
    V = 20000
    L = O.normal(59, (rows, V), 0.0, 3.0, F32).view(np.float32).copy()
    keep = []
    for r in range(rows):
        x = np.sort(L[r])[::-1]
        e32 = np.exp(x - x[0])
        p64 = softmax(x.astype(np.float64))
        c32 = np.searchsorted(np.cumsum(e32 / e32.sum()), np.float32(0.9)) + 1
        c64 = np.searchsorted(np.cumsum(p64), np.float64(np.float32(0.9))) + 1
        keep.append(c32 == c64)   # rows whose cut the two precisions place alike
    assert sum(keep) >= rows - 2
    want = O.sample_rows(L, np.argmax(L, axis=1), 0, 1.0, 0.9, 0.0)
    ids, probs, n = prims.sample_rows(torch.from_numpy(L).cuda(), 0, 1.0, 0.9, 0.0)
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        if not keep[r]:
            continue
        wi, wp = want[r]
        assert n[r] == len(wi), (r, n[r], len(wi))
        assert np.array_equal(ids[r, :n[r]], wi), r
        assert np.abs(probs[r, :n[r]].astype(np.float64) - wp).max() <= 2e-6, r


@pytest.mark.parametrize("case", range(8))
def test_sample_rows_split_random(prims, case):
    """seeded random configurations through the split path (sorted outputs, no
    top_k cut): row counts giving 8 down to 2 work-groups per row, widths off
    whole groups, spreads, -inf and NaN entries, top_p / min_p / temperature;
    rows whose cut float32 and f64 place apart are skipped (asserted rare)"""
    import torch
    rng = np.random.default_rng(1000 + case)
    rows = int(rng.choice([1, 7, 33, 64, 100]))
    V = int(rng.integers(16384, 60000))
    sigma = float(rng.choice([1.0, 3.0, 6.0]))
    top_k = int(rng.choice([0, V, V + 5]))
    top_p = float(rng.choice([0.5, 0.9, 0.99]))
    min_p = float(rng.choice([0.0, 0.02]))
    temp = float(rng.choice([0.5, 1.0, 1.5]))
    L = (rng.standard_normal((rows, V)) * sigma).astype(np.float32)
    L[rng.random((rows, V)) < 0.01] = -np.inf
    if case % 2:
        L[rng.random((rows, V)) < 0.001] = np.nan
    keep = []
    for r in range(rows):
        x = L[r][np.isfinite(L[r])]
        x = np.sort(x)[::-1]
        e32 = np.exp(x - x[0])
        p64 = softmax(x.astype(np.float64))
        c32 = np.searchsorted(np.cumsum(e32 / e32.sum()), np.float32(top_p)) + 1
        c64 = np.searchsorted(np.cumsum(p64), np.float64(np.float32(top_p))) + 1
        ok = c32 == c64 or min(c32, c64) > 4096  # (past 4096 the device leaves the row to the host)
        if min_p > 0.0:
            ok = ok and np.min(np.abs(p64 / p64[0] - np.float32(min_p))) > 1e-6
        keep.append(ok)
    assert sum(keep) >= rows - max(2, rows // 10), (rows, sum(keep))
    want = O.sample_rows(L, np.argmax(L, axis=1), top_k, temp, top_p, min_p)
    ids, probs, n = prims.sample_rows(torch.from_numpy(L).cuda(), top_k, temp, top_p, min_p)
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        if not keep[r]:
            continue
        wi, wp = want[r]
        if len(wi) > 4096:
            assert n[r] == -1, r
            continue
        assert n[r] == len(wi), (case, r, n[r], len(wi))
        assert np.array_equal(ids[r, :n[r]], wi), (case, r)
        assert np.abs(probs[r, :n[r]].astype(np.float64) - wp).max() <= 2e-6, (case, r)


def test_sample_rows_left_to_host(prims):
    """count -1: a nucleus of more than 4096 sorted candidates (flat logits), and a
    row holding +inf (the reference's probabilities are NaN there); other rows of
    the same call are served"""
    import torch
    V = 20000
    L = np.zeros((3, V), np.float32)
    L[0] = np.linspace(0.0, 0.01, V, dtype=np.float32)   # almost flat: nucleus ~ 0.95 V
    L[1, 5] = np.inf
    L[2] = np.linspace(0.0, 40.0, V, dtype=np.float32)   # steep: a short nucleus
    ids, probs, n = prims.sample_rows(torch.from_numpy(L).cuda(), 0, 1.0, 0.95, 0.0)
    n = n.cpu().numpy()
    assert n[0] == -1 and n[1] == -1
    (wi, wp), = O.sample_rows(L[2:3], [0], 0, 1.0, 0.95, 0.0)
    assert n[2] == len(wi)
    assert np.array_equal(ids.cpu().numpy()[2, :n[2]], wi)
