"""CPU: pins of the oracle that do not come from the reference's code.

Each check uses an independent formulation — numpy's own float16 cast,
integer-bit RNE, extended-precision (longdouble) evaluation, numpy/scipy
reductions and sorts, closed forms and invariants — chosen so that a dropped
rounding step, a wrong sign, a swapped operand or a wrong tie rule in the
oracle fails one of them. The ulp gates follow the reference's own
transcendental KATs (tests/fmath_test.cpp:54-185).
"""
import math

import numpy as np
import pytest

import oracle as O

F64, BF16, F16, F32 = O.F64, O.BF16, O.F16, O.F32
RNG = np.random.default_rng(2026)


# ----------------------------------------------------------------- rounding
def bf16_rne_bits(f32):
    """RNE of f32 values to bf16 bits by integer arithmetic on the pattern"""
    u = np.asarray(f32, np.float32).view(np.uint32).astype(np.uint64)
    upper, rem = u >> 16, u & 0xFFFF
    up = (rem > 0x8000) | ((rem == 0x8000) & ((upper & 1) == 1))
    out = (upper + up).astype(np.uint16)
    nan = np.isnan(np.asarray(f32, np.float32))
    return np.where(nan, np.uint16(0x7FC0), out)


def test_16bit_patterns_round_trip():
    bits = np.arange(65536, dtype=np.uint16)
    for dt in (BF16, F16):
        v = O.to_f64(bits, dt)
        ok = ~np.isnan(v)
        assert np.array_equal(O.from_f64(v[ok], dt), bits[ok])


def test_f16_decode_matches_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    v = O.to_f64(bits, F16)
    ref = bits.view(np.float16).astype(np.float64)
    ok = ~np.isnan(ref)
    assert np.array_equal(np.isnan(v), ~ok)
    assert np.array_equal(v[ok], ref[ok])


def test_bf16_rounding_double_rounding_chain():
    """f64 -> f32 (RNE) -> bf16 (RNE), NaN -> 0x7FC0 (src/rounding.hpp:64-75)"""
    x = np.concatenate([RNG.normal(0, 1, 200000) * np.exp2(RNG.integers(-140, 120, 200000)),
                        [0.0, -0.0, np.inf, -np.inf, np.nan, 3.4e38, 3.39e38]])
    # exact bf16 midpoints and values a hair off them: the double-rounding traps
    u = np.float32(RNG.normal(0, 1, 20000)).view(np.uint32)
    mid = ((u & 0xFFFF0000) | 0x8000).view(np.float32).astype(np.float64)
    x = np.concatenate([x, mid, mid * (1 + 2.0**-30), mid * (1 - 2.0**-30), mid * (1 + 2.0**-60)])
    with np.errstate(over="ignore"):
        ref = bf16_rne_bits(x.astype(np.float32))
    assert np.array_equal(O.from_f64(x, BF16), ref)


def test_f16_rounding_matches_numpy_cast():
    """f64 -> f32 -> f16 RNE with subnormals and overflow to inf (src/rounding.hpp:78-123)
    against numpy's own float32 -> float16 cast"""
    x = np.concatenate([RNG.normal(0, 1, 200000) * np.exp2(RNG.integers(-30, 18, 200000)),
                        [65504.0, 65519.0, 65520.0, 2.0**-24, 2.0**-25, 3 * 2.0**-26, 0.0, -0.0]])
    u = np.float32(RNG.normal(0, 1, 20000) * 2.0**-16).view(np.uint32)
    mid = ((u & 0xFFFFE000) | 0x1000).view(np.float32).astype(np.float64)
    x = np.concatenate([x, mid, mid * (1 + 2.0**-30)])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(O.from_f64(x, F16), ref)


def test_nan_canonicalization():
    assert O.from_f64(np.array([np.nan, -np.nan]), BF16).tolist() == [0x7FC0, 0x7FC0]
    f16 = O.from_f64(np.array([np.nan, -np.nan]), F16)
    assert (f16[0] & 0x7FFF) == 0x7E00 and (f16[1] & 0x7FFF) == 0x7E00


# -------------------------------------------------------------------- fmath
def ulps(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    ia = a.view(np.int64)
    ib = b.view(np.int64)
    oa = np.where(ia < 0, np.int64(-(2**63)) + 1 - ia, ia)
    ob = np.where(ib < 0, np.int64(-(2**63)) + 1 - ib, ib)
    d = np.abs(oa - ob)
    return np.where(a == b, 0, d)


@pytest.mark.parametrize("fn,ref,lo,hi,gate", (
    (O.exp, np.exp, -745.0, 700.0, 4), (O.exp, np.exp, -30.0, 0.0, 4),
    (O.log, np.log, 1e-12, 1e12, 4), (O.log, np.log, 0.5, 2.0, 4),
    (O.tanh, np.tanh, -30.0, 30.0, 4), (O.tanh, np.tanh, -1.0, 1.0, 4),
    (O.expm1, np.expm1, -50.0, 50.0, 4),
    (O.sin, np.sin, 0.0, 1.6e6, 4), (O.cos, np.cos, 0.0, 1.6e6, 4),
    (O.sin, np.sin, -8.0, 8.0, 4), (O.cos, np.cos, -8.0, 8.0, 4),
))
def test_fmath_ulp_vs_libm(fn, ref, lo, hi, gate):
    """tests/fmath_test.cpp:54-185: core functions within 4 ulp of glibc"""
    x = RNG.uniform(lo, hi, 400000)
    assert ulps(fn(x), ref(x)).max() <= gate


def test_pow_ulp_and_rope_grid():
    a = RNG.uniform(1.5, 2e6, 200000)
    b = RNG.uniform(-1.5, 1.5, 200000)
    y = np.array([O.pow_(ai, np.array([bi]))[0] for ai, bi in zip(a[:20000], b[:20000])])
    assert ulps(y, np.power(a[:20000], b[:20000])).max() <= 16
    for theta in (1e4, 1e6, 5e5):
        for dim in (128, 256, 512):
            e = -np.arange(0, dim, 2) / dim
            assert ulps(O.pow_(theta, e), np.power(theta, e)).max() <= 16


def test_fmath_identities():
    z = np.array([0.0])
    assert O.exp(z)[0] == 1.0 and O.cos(z)[0] == 1.0 and O.sin(z)[0] == 0.0
    assert O.tanh(z)[0] == 0.0 and O.log(np.array([1.0]))[0] == 0.0 and O.pow_(7.0, z)[0] == 1.0
    assert O.exp(np.array([-800.0]))[0] == 0.0
    assert O.tanh(np.array([50.0, -50.0])).tolist() == [1.0, -1.0]


# ----------------------------------------------------------- silu / sigmoid
def ld_silu(x):
    x = np.asarray(x, np.longdouble)
    return x / (1 + np.exp(-x))


def test_silu_sigmoid_table_all_bf16_inputs():
    """rnd(silu(g)) and rnd(sigmoid(g)) for every finite bf16 g equal the
    extended-precision value rounded the twin's way (f64 -> f32 -> bf16)"""
    bits = np.arange(65536, dtype=np.uint16)
    g = O.to_f64(bits, BF16)
    ok = np.isfinite(g) & (np.abs(g) < 1e30)
    with np.errstate(over="ignore"):
        ref_silu = O.from_f64(np.asarray(ld_silu(g[ok]), np.float64), BF16)
        ref_sig = O.from_f64(np.asarray(1 / (1 + np.exp(-np.asarray(g[ok], np.longdouble))), np.float64), BF16)
    assert np.array_equal(O.from_f64(O.silu(g[ok]), BF16), ref_silu)
    assert np.array_equal(O.from_f64(O.sigmoid(g[ok]), BF16), ref_sig)


def test_swiglu_twin_composition():
    """rnd(rnd(silu(g)) * u): the product of two bf16 values is exact in f32,
    so numpy's f32 multiply followed by an integer RNE must agree bit for bit"""
    g = O.rnd(RNG.normal(0, 2, 200000), BF16)
    u = O.rnd(RNG.normal(0, 2, 200000), BF16)
    s = O.to_f64(O.from_f64(O.silu(g), BF16), BF16).astype(np.float32)
    ref = bf16_rne_bits(s * u.astype(np.float32))
    assert np.array_equal(O.from_f64(O.swiglu(g, u, BF16), BF16), ref)
    # f64 mode is the unrounded product
    assert np.array_equal(O.swiglu(g, u, F64), O.silu(g) * u)


def test_residual_add_twin():
    h = O.rnd(RNG.normal(0, 1, 200000), BF16)
    x = O.rnd(RNG.normal(0, 3, 200000) * np.exp2(RNG.integers(-20, 20, 200000)), BF16)
    ref = bf16_rne_bits(h.astype(np.float32) + x.astype(np.float32))
    assert np.array_equal(O.from_f64(O.residual_add(h, x, BF16), BF16), ref)


def test_sigmoid_gate_twin():
    pv = O.rnd(RNG.normal(0, 1, 100000), BF16)
    gt = O.rnd(RNG.normal(0, 2, 100000), BF16)
    sg = O.to_f64(O.from_f64(O.sigmoid(gt), BF16), BF16).astype(np.float32)
    assert np.array_equal(O.from_f64(O.sigmoid_gate(pv, gt, BF16), BF16), bf16_rne_bits(pv.astype(np.float32) * sg))


def test_scale_uses_f32_scalar():
    x = O.rnd(RNG.normal(0, 1, 100000), BF16)
    ref = bf16_rne_bits(x.astype(np.float32) * np.float32(3.87))
    assert np.array_equal(O.from_f64(O.scale(x, 3.87, BF16), BF16), ref)
    xf = O.rnd(RNG.normal(0, 1, 100000), F32)
    assert np.array_equal(O.scale(xf, 3.87, F32), (xf.astype(np.float32) * np.float32(3.87)).astype(np.float64))


# -------------------------------------------------------------------- norms
def test_mean_sq_exact_on_integers():
    """small integers: every partial sum is exact, so any order gives sum(x^2)/n"""
    x = RNG.integers(-1000, 1000, (50, 777)).astype(np.float64)
    assert np.array_equal(O.mean_sq(x), (x * x).sum(1) / 777)


@pytest.mark.parametrize("kind", (O.CENTERED, O.PLAIN, O.WEIGHTLESS))
def test_rmsnorm_f64_vs_extended(kind):
    x = RNG.normal(0, 1, (64, 5120))
    w = RNG.normal(1, 0.05, 5120)
    y = O.rmsnorm_rows(kind, x, w, 1e-6, F64)
    xl = x.astype(np.longdouble)
    rs = 1 / np.sqrt((xl * xl).mean(1, keepdims=True) + np.longdouble(1e-6))
    ref = xl * rs
    if kind == O.CENTERED:
        ref = ref * (1 + w.astype(np.longdouble))
    elif kind == O.PLAIN:
        ref = ref * w.astype(np.longdouble)
    rel = np.abs((y - ref) / ref).astype(np.float64)
    assert rel.max() < 1.5e-15  # a few ulp: the row sum, sqrt, division and two products


@pytest.mark.parametrize("kind", (O.CENTERED, O.PLAIN, O.WEIGHTLESS))
@pytest.mark.parametrize("dt", (BF16, F16, F32))
def test_bf16exec_norm_rows_is_the_f64_norm_rounded_once(kind, dt):
    """bf16exec's norm_rows (src/bf16exec.hpp:398-421) sums in index order, the twin in
    mean_sq's; on integer rows both sums are exact, so its output must be the pinned f64
    norm rounded once to dt (a wrong weight form, rounding or eps shows up here)"""
    X = RNG.integers(-40, 41, (13, 200)).astype(np.float64)
    X[3] = 0.0
    w = O.rnd(RNG.normal(1, 0.05, 200), BF16)
    got = O.norm_rows_mixed(kind, X, w, 1e-6, dt)
    ref = O.rnd(O.rmsnorm_rows(kind, X, w, 1e-6, F64), dt)
    assert np.array_equal(got, ref)


def test_rmsnorm_invariants():
    x = RNG.normal(0, 1, (16, 640))
    w = RNG.normal(1, 0.1, 640)
    y = O.rmsnorm_rows(O.PLAIN, x, w, 0.0, F64)
    # scale invariance (eps = 0) and row independence
    assert np.allclose(O.rmsnorm_rows(O.PLAIN, 8 * x, w, 0.0, F64), y, rtol=0, atol=1e-15)
    assert np.array_equal(O.rmsnorm_rows(O.PLAIN, x[::-1], w, 0.0, F64), y[::-1])
    # unit rms with w = 1
    y1 = O.rmsnorm_rows(O.WEIGHTLESS, x, None, 0.0, F64)
    assert np.allclose((y1 * y1).mean(1), 1.0, rtol=1e-14)


# --------------------------------------------------------------------- rope
def test_rope_table_vs_numpy_f64():
    theta, dim, T = 1e6, 128, 4096
    c, s = O.rope_table(theta, dim, T, F64)
    inv = 1.0 / np.power(theta, np.arange(0, dim, 2) / dim)
    ang = np.arange(T)[:, None] * inv[None, :]
    assert np.abs(c - np.cos(ang)).max() < 1e-12
    assert np.abs(s - np.sin(ang)).max() < 1e-12


def test_rope_rotation_f64_is_a_rotation():
    c, s = O.rope_table(1e4, 64, 100, F64)
    x = RNG.normal(0, 1, (100, 3, 64))
    y = O.apply_rope(x, c, s, np.arange(100), F64)
    # norm of each (lo, hi) pair is preserved and position 0 is the identity
    assert np.allclose(np.hypot(y[..., :32], y[..., 32:]), np.hypot(x[..., :32], x[..., 32:]), rtol=1e-14)
    assert np.array_equal(y[0], x[0])


def test_rope_twin_three_roundings():
    """x' = rnd(rnd(lo*c) + rnd(-hi*s)): bf16 products are exact in f32"""
    c, s = O.rope_table(1e6, 128, 64, BF16)
    x = O.rnd(RNG.normal(0, 1, (64, 2, 128)), BF16)
    y = O.apply_rope(x, c, s, np.arange(64), BF16)
    lo, hi = x[..., :64].astype(np.float32), x[..., 64:].astype(np.float32)
    cc, ss = c[:, None, :].astype(np.float32), s[:, None, :].astype(np.float32)

    def r(v):
        return O.to_f64(bf16_rne_bits(v), BF16).astype(np.float32)
    ref_lo = bf16_rne_bits(r(lo * cc) + r(-(hi * ss)))
    ref_hi = bf16_rne_bits(r(hi * cc) + r(lo * ss))
    got = O.from_f64(y, BF16)
    assert np.array_equal(got[..., :64], ref_lo) and np.array_equal(got[..., 64:], ref_hi)


# ------------------------------------------------------------------ softmax
def np_softmax(s, vis):
    s = np.where(vis, s, -np.inf)
    m = s.max(-1, keepdims=True)
    e = np.where(vis, np.exp(s - m), 0.0)
    return e / e.sum(-1, keepdims=True)


@pytest.mark.parametrize("mask,window,q0", ((O.MASK_NONE, 0, 0), (O.MASK_CAUSAL, 0, 0), (O.MASK_CAUSAL, 0, 100),
                                            (O.MASK_WINDOW, 50, 200), (O.MASK_BIWINDOW, 30, 10),
                                            (O.MASK_BIWINDOW, 30, 280)))
def test_softmax_vs_numpy(mask, window, q0):
    heads, q, k = 3, 64, 300
    x = O.rnd(RNG.normal(0, 30, (heads, q, k)), F32)
    scale = 1 / math.sqrt(128)
    y = O.softmax_rows(x, scale, mask, window, q0, 0.0, F32, F64)
    s = (x.astype(np.float32) * np.float32(scale)).astype(np.float64)
    qpos = q0 + np.arange(q)[:, None]
    j = np.arange(k)[None, :]
    vis = np.ones((q, k), bool) if mask in (O.MASK_NONE, O.MASK_BIWINDOW) else (j <= qpos)
    if mask == O.MASK_WINDOW:
        vis &= j > qpos - window
    if mask == O.MASK_BIWINDOW:
        vis &= (j >= qpos - window) & (j <= qpos + window)
    ref = np_softmax(s, vis[None])
    assert np.all(y[:, ~vis] == 0.0)
    v = np.broadcast_to(vis, y.shape) & (ref > 1e-300)
    assert np.abs(y[v] / ref[v] - 1).max() < 1e-13
    live = vis.any(-1)  # rows with no visible key are all zero
    assert np.abs(y.sum(-1)[:, live] - 1).max() < 1e-13
    assert np.all(y.sum(-1)[:, ~live] == 0.0)


def test_softmax_softcap_and_16bit_scores():
    x = O.rnd(RNG.normal(0, 60, (2, 8, 64)), BF16)
    y = O.softmax_rows(x, 0.125, O.MASK_NONE, 0, 0, 30.0, BF16, F64)
    # the eager chain with bf16 materializations at each step
    s = O.rnd(x * np.float64(np.float32(0.125)), BF16)
    s = O.softcap(s, 1.0, 30.0, BF16)
    ref = np_softmax(s, np.ones(s.shape, bool))
    assert np.abs(y / ref - 1).max() < 1e-13


def test_softmax_shift_invariance():
    x = RNG.normal(0, 2, (1, 4, 100))
    a = O.softmax_rows(x, 1.0, O.MASK_NONE, 0, 0, 0.0, F64, F64)
    b = O.softmax_rows(x + 7.0, 1.0, O.MASK_NONE, 0, 0, 0.0, F64, F64)
    assert np.abs(a / b - 1).max() < 1e-13


def test_softmax_f64_scores_vs_numpy():
    x = RNG.normal(0, 4, (2, 16, 200))
    y = O.softmax_rows(x, 0.3, O.MASK_CAUSAL, 0, 150, 0.0, F64, F64)
    qpos = 150 + np.arange(16)[:, None]
    vis = np.arange(200)[None, :] <= qpos
    ref = np_softmax(x * 0.3, vis[None])
    v = np.broadcast_to(vis, y.shape)
    assert np.all(y[~v] == 0.0)
    assert np.abs(y[v] / ref[v] - 1).max() < 1e-13


def _compat(x, scale=1.0, mask=O.MASK_NONE, window=0, q0=0):
    return O.softmax_rows(np.asarray(x, np.float64), scale, mask, window, q0, 0.0, F64 | O.F32_COMPAT, F64)


def test_softmax_f32_compat_known_answers():
    """The --hf-f32-compat softmax (muse_glimmer.hpp:856-870) on rows whose
    answer only its exact chain gives."""
    # 1. the sum is one f32 chain in ascending key order: with e = float(exp(s))
    #    just below 2^-24, 1 + e rounds back to 1 at every step, so the row
    #    [0, s, ..., s] keeps sum32 = 1 and p[0] = 1 exactly; an f64 sum, a
    #    pairwise sum or the descending order gives sum32 > 1
    s32 = np.float32(-24 * math.log(2))
    while O.exp(np.array([float(s32)]))[0].astype(np.float32) >= np.float32(2.0 ** -24):
        s32 = np.nextafter(s32, np.float32(-np.inf))
    e = float(np.float32(O.exp(np.array([float(s32)]))[0]))
    assert 2.0 ** -25 < e < 2.0 ** -24
    n = 1000
    row = np.full(n + 1, float(s32))
    row[0] = 0.0
    y = _compat(row[None, None, :])[0, 0]
    assert y[0] == 1.0 and np.all(y[1:] == e)
    #    the reversed row adds the small terms first: sum32 > 1 + (n - 1) e
    y = _compat(row[::-1].copy()[None, None, :])[0, 0]
    assert y[-1] < 1.0 and abs(y[-1] * (1 + n * e) - 1) < 1e-6
    # 2. the max and the differences are f32: scores that differ below f32
    #    resolution become equal and split the mass exactly
    y = _compat([[[1.0 + 1e-12, 1.0, 1.0 - 1e-12]]])[0, 0]
    assert np.all(y == float(np.float32(1.0 / 3.0)))
    p64 = O.softmax_rows(np.array([[[1.0 + 1e-12, 1.0]]]), 1.0, O.MASK_NONE, 0, 0, 0.0, F64, F64)[0, 0]
    assert p64[0] != p64[1]
    # 3. masked keys exactly 0, f32-valued outputs, within f32 error of f64
    x = RNG.normal(0, 3, (2, 40, 120))
    y = _compat(x, 0.7, O.MASK_WINDOW, 17, 60)
    ref = O.softmax_rows(x, 0.7, O.MASK_WINDOW, 17, 60, 0.0, F64, F64)
    assert np.array_equal(y, y.astype(np.float32).astype(np.float64))
    assert np.all((y == 0.0) == (ref == 0.0))
    nz = ref > 1e-30
    assert np.abs(y[nz] / ref[nz] - 1).max() < 1e-5
    assert not np.array_equal(y, ref)


# --------------------------------------------------------------------- Q8_0
def test_dequant_vs_numpy():
    qs = O.int8_uniform(1, (64, 256), -128, 127)
    d = O.uniform(2, (64, 8), 1e-5, 2e-2, F16)
    ref64 = qs.astype(np.float64) * np.repeat(d.view(np.float16).astype(np.float64), 32, axis=1)
    for dt in (BF16, F16, F32):
        got = O.from_f64(O.dequant_q8_0(qs, d, dt), dt)
        if dt == BF16:
            want = bf16_rne_bits(ref64.astype(np.float32))
        elif dt == F16:
            want = ref64.astype(np.float32).astype(np.float16).view(np.uint16)
        else:
            want = ref64.astype(np.float32)
        assert np.array_equal(got, want)


def test_quantize_invariants():
    """up_w (src/gpu/gpu_engine.cpp:2722-2755): |q| <= 127, the block maximum maps
    to +-127, |x - q d| <= d/2 up to the f16 rounding of d, and the scale is the
    f16 cast of amax/127 (parity against llama.cpp itself is unpinned)"""
    w = O.normal(3, (32, 512), 0, 1, BF16)
    qs, d = O.quantize_q8_0(w)
    x = O.to_f64(w, BF16).reshape(32, 16, 32)
    q = qs.astype(np.float64).reshape(32, 16, 32)
    amax = np.abs(x).max(-1)
    assert np.abs(qs).max() <= 127
    assert np.array_equal(d, (amax.astype(np.float32) / np.float32(127)).astype(np.float16).view(np.uint16))
    d32 = (amax.astype(np.float32) / np.float32(127)).astype(np.float64)[..., None]
    assert np.all(np.abs(q).max(-1) == 127)
    # q rounds x / d with the f32 d (half away from zero); the stored f16 d differs from it
    # by at most 2^-11 relative
    assert np.all(np.abs(x - q * d32) <= d32 * (0.5 + 1e-5))  # x*id is an f32 product
    dd = d.view(np.float16).astype(np.float64)[..., None]
    assert np.all(np.abs(dd - d32) <= d32 * 2.0**-11)


def test_quantize_ties_round_half_away_from_zero():
    """up_w's q = (int8)lround(x * id) (src/gpu/gpu_engine.cpp:2722-2755): a product
    that lands exactly on k + 1/2 rounds away from zero, to sign(x) (k + 1). The
    blocks are built so that id is a power of two and x * id is exact: amax 127
    gives d = 1, amax 63.5 gives d = 1/2 (id = 2), amax 254 gives d = 2 (id = 1/2);
    every other element is a tie at that scale. Half-to-even (rint, np.round) would
    give 0 for 0.5, 2 for 2.5 and -2 for -2.5 and fails here."""
    ks = np.array([0, 1, 2, 3, 4, 5, 62, 125, 0, 1, 2, 7, 9, 100, 126, 64,
                   0, 3, 6, 11, 20, 40, 80, 99, 1, 2, 4, 8, 16, 32, 120], np.int64)
    sign = np.where(np.arange(ks.size) % 3 == 1, -1, 1)
    blocks = []
    for amax, idv in ((127.0, 1.0), (63.5, 2.0), (254.0, 0.5)):
        x = np.concatenate([[amax], sign * (ks + 0.5) / idv]).astype(np.float32)  # x * id = sign (k + 1/2)
        b = x.view(np.uint32)
        assert np.all((b & 0xffff) == 0) and np.abs(x).max() == amax  # exact bf16 values
        blocks.append((b >> 16).astype(np.uint16))
    qs, d = O.quantize_q8_0(np.stack(blocks))
    assert np.array_equal(d.view(np.float16).astype(np.float64).ravel(), [1.0, 0.5, 2.0])
    away = np.concatenate([[127], sign * (ks + 1)])
    even = np.concatenate([[127], np.round(sign * (ks + 0.5)).astype(np.int64)])
    assert not np.array_equal(away, even)
    for r in range(3):
        assert np.array_equal(qs[r].astype(np.int64), away), r


# -------------------------------------------------------------------- vocab
def test_vocab_vs_numpy():
    from scipy.special import logsumexp
    L = O.rnd(RNG.normal(0, 4, (8, 20000)), F32)
    L[1, ::7] = -np.inf
    L[2] = np.round(L[2])  # ties
    lse, am, ti, tv = O.vocab_reduce(L, 64)
    for r in range(8):
        fin = np.isfinite(L[r])
        assert abs(lse[r] - logsumexp(L[r][fin])) <= 1e-13 * abs(lse[r])
        assert am[r] == int(np.argmax(L[r]))
        order = np.lexsort((np.arange(L.shape[1]), -L[r]))[:64]
        assert np.array_equal(ti[r], order) and np.array_equal(tv[r], L[r][order])


def test_vocab_special_values():
    """NaN ranks below -inf, -0 == +0 (ties by index), lse over finite entries,
    argmax = first maximum of the non-NaN entries unless index 0 is NaN"""
    from scipy.special import logsumexp
    L = O.rnd(RNG.normal(0, 4, (5, 3000)), F32)
    L[0, 5::97] = np.nan
    L[1, [1234, 2000]] = np.inf
    L[1, 7::50] = np.nan
    L[2] = -np.abs(L[2])
    L[2, 3::11] = 0.0
    L[2, 8::13] = -0.0
    L[3, :] = np.nan
    L[3, 100::300] = 1.5
    L[4, 0] = np.nan
    lse, am, ti, tv = O.vocab_reduce(L, 64)
    idx = np.arange(L.shape[1])
    for r in range(5):
        fin = np.isfinite(L[r])
        if fin.any():
            assert abs(lse[r] - logsumexp(L[r][fin])) <= 1e-13 * abs(lse[r])
        nan = np.isnan(L[r])
        assert am[r] == (0 if nan[0] else int(np.nanargmax(L[r])))
        order = np.lexsort((idx, -np.where(nan, 0.0, L[r]), nan))[:64]
        assert np.array_equal(ti[r], order)
        assert np.array_equal(np.isnan(tv[r]), nan[order])


def test_vocab_all_masked_row():
    L = np.full((1, 100), -np.inf)
    lse, am, ti, tv = O.vocab_reduce(L, 4)
    assert lse[0] == -np.inf and am[0] == 0 and ti[0].tolist() == [0, 1, 2, 3]


# --------------------------------------------------------------- generators
def test_generator_deterministic_and_distributed():
    a = O.normal(5, (1 << 18,), 1.0, 0.05, F64)
    b = O.normal(5, (1 << 18,), 1.0, 0.05, F64)
    assert np.array_equal(a, b)
    assert abs(a.mean() - 1.0) < 1e-3 and abs(a.std() - 0.05) < 1e-3
    q = O.int8_uniform(9, (1 << 18,))
    assert q.min() == -127 and q.max() == 127 and abs(q.mean()) < 1.0
