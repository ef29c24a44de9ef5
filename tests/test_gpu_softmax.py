"""GPU parity: scaled, masked row softmax.

Reference: the softmax of attention_forward (src/muse_glimmer.hpp:828-885) as a
row operator (oracle/oracle.cpp or_softmax_rows); softcap in apply_output_tail's
op order (920-943). Gates: bf16 probabilities within 1 ulp of the twin (f64
internals, one rounding); f32 probabilities within 1e-6 relative of the f64
oracle; masked probabilities exactly 0.
"""
import math

import numpy as np
import pytest

import oracle as O
from util import BF16, F16, F32, from_dev, same_bits, storage, to_dev, ulp_diff16

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128.0)


def run(prims, heads, q, kc, dt_in=F32, dt_out=BF16, mask=O.MASK_CAUSAL, window=0, q_pos0=0,
        softcap=0.0, seed=8, std=3.0):
    xs, x = storage(seed, (heads, q, kc), dt_in, 0.0, std)
    dx = to_dev(xs, dt_in)
    dy = to_dev(np.zeros((heads, q, kc), np.float32 if dt_out == F32 else np.uint16), dt_out)
    prims.softmax_rows(dx, dy, SCALE, mask, window, q_pos0, softcap)
    y = from_dev(dy, dt_out)
    ref = O.softmax_rows(x, SCALE, mask, window, q_pos0, softcap, dt_in, O.F64)
    return y, ref


def visible(heads, q, kc, mask, window, q_pos0):
    qpos = q_pos0 + np.arange(q)[:, None]
    j = np.arange(kc)[None, :]
    v = np.ones((q, kc), bool)
    if mask == 3:
        v &= (j >= qpos - window) & (j <= qpos + window)
        return np.broadcast_to(v, (heads, q, kc))
    if mask >= 1:
        v &= j <= qpos
    if mask == 2:
        v &= j > qpos - window
    return np.broadcast_to(v, (heads, q, kc))


def check(y, ref, dt_out, vis, max_frac=2e-3):
    assert np.all(O.to_f64(y, dt_out)[~vis] == 0.0), "masked probability not exactly 0"
    if dt_out == F32:
        yv = y.astype(np.float64)[vis]
        rv = ref[vis]
        rel = np.abs(yv - rv) / rv
        i = int(np.argmax(rel))
        assert rel.max() <= 1e-6, (rel.max(), float(yv[i]), float(rv[i]), i)
        return 0
    d = ulp_diff16(y, O.from_f64(ref, dt_out))
    assert d.max() <= 1, d.max()
    frac = (d > 0).mean()
    assert frac <= max_frac, frac
    return int((d > 0).sum())


@pytest.mark.parametrize("dt_out", (BF16, F32, F16))
@pytest.mark.parametrize("mask", (O.MASK_NONE, O.MASK_CAUSAL))
def test_prefill_rows(prims, dt_out, mask):
    y, ref = run(prims, 8, 256, 256, dt_out=dt_out, mask=mask)
    check(y, ref, dt_out, visible(8, 256, 256, mask, 0, 0))


@pytest.mark.parametrize("kc", (2048, 1024, 512, 100, 8, 1))
def test_row_lengths(prims, kc):
    y, ref = run(prims, 3, 40, kc, q_pos0=kc - 40 if kc > 40 else 0)
    check(y, ref, BF16, visible(3, 40, kc, O.MASK_CAUSAL, 0, kc - 40 if kc > 40 else 0))


@pytest.mark.parametrize("dt_out", (BF16, F32))
def test_softcap(prims, dt_out):
    y, ref = run(prims, 4, 128, 1024, dt_out=dt_out, softcap=30.0, std=60.0)
    vis = visible(4, 128, 1024, O.MASK_CAUSAL, 0, 0)
    if dt_out == F32:
        # where a probability is off, how far off is the score it implies (in f32 ulps)?
        xs, x = storage(8, (4, 128, 1024), F32, 0.0, 60.0)
        s = O.softcap(O.rnd(x * np.float64(np.float32(SCALE)), F32), 1.0, 30.0, F32)
        s = np.where(vis, s, -np.inf)
        m = s.max(-1, keepdims=True)
        S = np.where(vis, np.exp(s - m), 0).sum(-1, keepdims=True)
        d_gpu = np.log(np.maximum(y.astype(np.float64), 1e-300) * S)
        dev = np.where(vis, (d_gpu - (s - m)) / np.spacing(np.abs(s).astype(np.float32)).astype(np.float64), 0)
        i = np.unravel_index(np.argmax(np.abs(dev)), dev.shape)
        print("worst implied score deviation (f32 ulps):", float(dev[i]), "at", i, "s =", float(s[i]), "m =", float(m[i[0], i[1], 0]))
    check(y, ref, dt_out, vis)


def test_window_mask(prims):
    y, ref = run(prims, 4, 64, 512, mask=O.MASK_WINDOW, window=100, q_pos0=300)
    check(y, ref, BF16, visible(4, 64, 512, O.MASK_WINDOW, 100, 300))


@pytest.mark.parametrize("dt_in", (BF16, F16))
def test_16bit_scores(prims, dt_in):
    y, ref = run(prims, 4, 64, 2048, dt_in=dt_in, q_pos0=1984)
    check(y, ref, BF16, visible(4, 64, 2048, O.MASK_CAUSAL, 0, 1984))


@pytest.mark.parametrize("dt_out", (BF16, F32))
def test_decode_split_rows(prims, dt_out):
    """Config 4 decode: [40, 1, 131072], every key visible (split path)."""
    y, ref = run(prims, 40, 1, 131072, dt_out=dt_out, q_pos0=131071)
    check(y, ref, dt_out, visible(40, 1, 131072, O.MASK_CAUSAL, 0, 131071))


def test_split_ragged_and_masked(prims):
    """split rows with k % 8 != 0 and a causal cut inside the row"""
    y, ref = run(prims, 3, 2, 9000 + 5, q_pos0=5000)
    check(y, ref, BF16, visible(3, 2, 9005, O.MASK_CAUSAL, 0, 5000))
    y, ref = run(prims, 2, 3, 20000, mask=O.MASK_WINDOW, window=7000, q_pos0=15000, dt_out=F32)
    check(y, ref, F32, visible(2, 3, 20000, O.MASK_WINDOW, 7000, 15000))


def test_split_many_rows(prims):
    """many split rows at once (1024 rows x 2 chunks): more work-groups than
    the device holds at a time"""
    y, ref = run(prims, 8, 128, 6000, q_pos0=5872)
    check(y, ref, BF16, visible(8, 128, 6000, O.MASK_CAUSAL, 0, 5872))


def test_split_repeat(prims):
    """split calls of different row counts and lengths in a row share the
    partials area: each gives the results a fresh call gives"""
    for heads, kc in ((40, 131072), (3, 9000), (40, 131072), (7, 70000), (3, 9000)):
        y, ref = run(prims, heads, 1, kc, q_pos0=kc - 1, seed=heads + kc)
        check(y, ref, BF16, visible(heads, 1, kc, O.MASK_CAUSAL, 0, kc - 1))


def test_split_two_kernel_nonfinite(prims):
    """split rows with a NaN or +inf score: NaN probabilities where the twin
    has them (canonical bits), exact zeros where masked, the rest untouched"""
    heads, q, kc = 3, 2, 9000
    xs, x = storage(9, (heads, q, kc), F32, 0.0, 3.0)
    x = x.copy()
    x[0, 0, 4321] = np.nan
    x[1, 1, 77] = np.inf
    xs = O.from_f64(x, F32)
    dx = to_dev(xs, F32)
    dy = to_dev(np.zeros((heads, q, kc), np.uint16), BF16)
    prims.softmax_rows(dx, dy, SCALE, O.MASK_CAUSAL, 0, 8990, 0.0)
    y = from_dev(dy, BF16)
    ref = O.from_f64(O.softmax_rows(x, SCALE, O.MASK_CAUSAL, 0, 8990, 0.0, F32, O.F64), BF16)
    bad = np.zeros((heads, q), bool)
    bad[0, 0] = bad[1, 1] = True
    assert np.array_equal(y[bad], ref[bad])
    d = ulp_diff16(y[~bad], ref[~bad])
    assert d.max() <= 1


@pytest.mark.parametrize("dt_out", (BF16, F32))
def test_bidirectional_window(prims, dt_out):
    """the drafter's bidirectional window (src/dflash.hpp:339-344): keys within
    `window` of the query position on both sides, clipped to the block"""
    y, ref = run(prims, 4, 16, 300, mask=O.MASK_BIWINDOW, window=40, q_pos0=-5, dt_out=dt_out)
    check(y, ref, dt_out, visible(4, 16, 300, O.MASK_BIWINDOW, 40, -5))
    y, ref = run(prims, 2, 8, 5000, mask=O.MASK_BIWINDOW, window=2100, q_pos0=2900, dt_out=dt_out)
    check(y, ref, dt_out, visible(2, 8, 5000, O.MASK_BIWINDOW, 2100, 2900))


def test_all_masked_row_is_zero(prims):
    """window rows with q_pos0 < 0 see no key at all: zeros, not NaN"""
    y, ref = run(prims, 1, 4, 64, mask=O.MASK_WINDOW, window=2, q_pos0=-10)
    assert np.all(O.to_f64(y, BF16) == 0.0)


@pytest.mark.parametrize("dt_out", (BF16, F16))
@pytest.mark.parametrize("mask", (O.MASK_WINDOW, O.MASK_BIWINDOW))
@pytest.mark.parametrize("kc,q_pos0", ((300, 330), (1000, 1030), (1800, 1830)))
def test_window_rows_past_the_block(prims, dt_out, mask, kc, q_pos0):
    """windowed rows whose window starts past the last key (q_pos >= kc + window - 1
    for WINDOW, q_pos - window > kc - 1 for BIWINDOW) see no key: their clamped
    range has lo > hi. The fast path (f32 scores, 16-bit probabilities) must
    write zeros there, not 1/kc, while the rows before them stay exact; kc is
    not a multiple of 512 (nor of 8 for kc = 300)."""
    y, ref = run(prims, 3, 16, kc, dt_out=dt_out, mask=mask, window=40, q_pos0=q_pos0)
    vis = visible(3, 16, kc, mask, 40, q_pos0)
    empty = ~vis.any(-1)
    assert empty.any() and (~empty).any()
    assert np.all(O.to_f64(y, dt_out)[empty] == 0.0)
    check(y, ref, dt_out, vis)


@pytest.mark.parametrize("kc", (2048, 1500, 512))
def test_softcap_fast_rows(prims, kc):
    """softcap 30 on the fast path (f32 scores, bf16 out) at every row-length
    class, scores spread so that the cap bends them (std 60 -> |s| up to ~25)"""
    y, ref = run(prims, 4, 64, kc, softcap=30.0, std=60.0, q_pos0=kc - 64)
    check(y, ref, BF16, visible(4, 64, kc, O.MASK_CAUSAL, 0, kc - 64))


@pytest.mark.parametrize("cap,std", ((1.0, 3.0), (-30.0, 60.0), (1048576.0, 60.0), (2.0 ** 21, 60.0), (0.5, 3.0)))
def test_softcap_fast_rows_other_caps(prims, cap, std):
    """the fast capped score at the ends of its range (|cap| = 1 and 2^20), at a
    negative cap, and caps outside it (2^21, 0.5) that take the accurate kernel:
    all within 1 bf16 ulp of the twin's chain with that cap"""
    y, ref = run(prims, 4, 64, 2048, softcap=cap, std=std, q_pos0=2048 - 64)
    check(y, ref, BF16, visible(4, 64, 2048, O.MASK_CAUSAL, 0, 2048 - 64))


def test_softcap_split_rows(prims):
    """softcap 30 on the split path (rows longer than 2048 keys), bf16 and f32 out"""
    y, ref = run(prims, 3, 2, 9001, softcap=30.0, std=60.0, q_pos0=8990)
    check(y, ref, BF16, visible(3, 2, 9001, O.MASK_CAUSAL, 0, 8990))
    y, ref = run(prims, 2, 1, 20000, softcap=30.0, std=60.0, q_pos0=19999, dt_out=F32)
    check(y, ref, F32, visible(2, 1, 20000, O.MASK_CAUSAL, 0, 19999))


def test_softcap_nonfinite(prims):
    """+-inf scores cap to +-30 (finite); a NaN score makes its row NaN"""
    heads, q, kc = 2, 4, 2048
    xs, x = storage(11, (heads, q, kc), F32, 0.0, 3.0)
    x = x.copy()
    x[0, 0, 100] = np.inf
    x[0, 1, 5] = -np.inf
    x[1, 2, 2000] = np.nan
    xs = O.from_f64(x, F32)
    dy = to_dev(np.zeros((heads, q, kc), np.uint16), BF16)
    prims.softmax_rows(to_dev(xs, F32), dy, SCALE, O.MASK_NONE, 0, 0, 30.0)
    y = from_dev(dy, BF16)
    ref = O.from_f64(O.softmax_rows(x, SCALE, O.MASK_NONE, 0, 0, 30.0, F32, O.F64), BF16)
    nan = np.zeros((heads, q), bool)
    nan[1, 2] = True
    assert np.array_equal(y[nan], ref[nan])
    assert ulp_diff16(y[~nan], ref[~nan]).max() <= 1


def test_config4_softcap_full(prims):
    """Config 4's softcap variant at full size: f32 [40, 2048, 2048] ~ N(0, 3),
    1/sqrt(128), causal, tanh softcap 30.0, bf16 out"""
    y, ref = run(prims, 40, 2048, 2048, softcap=30.0)
    n = check(y, ref, BF16, visible(40, 2048, 2048, O.MASK_CAUSAL, 0, 0))
    print(f"config4 softcap 30: {n} of {y.size} probabilities differ from the twin by 1 ulp")


def test_config4_full(prims):
    """Config 4 prefill at full size: f32 [40, 2048, 2048] ~ N(0, 3), causal, bf16 out."""
    y, ref = run(prims, 40, 2048, 2048)
    n = check(y, ref, BF16, visible(40, 2048, 2048, O.MASK_CAUSAL, 0, 0))
    print(f"config4: {n} of {y.size} probabilities differ from the twin by 1 ulp")


def test_rows_sum_to_one(prims):
    y, _ = run(prims, 4, 64, 2048, dt_out=F32)
    s = y.astype(np.float64).sum(-1)
    assert np.abs(s - 1).max() < 1e-5


def test_errors(prims):
    import mgprims
    import torch
    x = torch.zeros((1, 1, 64), dtype=torch.float64, device="cuda:0")
    y = torch.zeros((1, 1, 64), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(mgprims.MgError, match="f64 probabilities"):
        prims.softmax_rows(x, y, 1.0)
    # the compat flag goes with f64 scores only
    xb = torch.zeros((1, 1, 64), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(mgprims.MgError, match="input dtype"):
        prims.softmax_rows(xb, y, 1.0, f32_compat=True)
