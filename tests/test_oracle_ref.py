"""CPU: the oracle restatement against oracle/_ref — the reference's own code
compiled from /root/reference (tests skip where it is not built, e.g. on a
machine without the reference) — on fresh random inputs, bitwise."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.skipif(not O.Ref.available(), reason="oracle/_ref not built (needs /root/reference)")
F64, BF16, F16 = O.F64, O.BF16, O.F16
RNG = np.random.default_rng(99)


@pytest.fixture(scope="module")
def R():
    return O.Ref()


def eq(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.array_equal(a.view(np.uint64), b.view(np.uint64))


def test_fmath(R):
    x = np.concatenate([RNG.uniform(-745, 709, 100000), RNG.normal(0, 5, 100000)])
    for n in ("exp", "tanh", "sin", "cos", "silu", "sigmoid"):
        assert eq(getattr(O, n)(x), R.vec(f"ok_{n}v", x)), n
    e = RNG.uniform(-1.5, 1.5, 20000)
    assert eq(O.pow_(12345.678, e), R.pow_(12345.678, e))


def test_rounding(R):
    x = RNG.normal(0, 1, 300000) * np.exp2(RNG.integers(-150, 130, 300000))
    for dt in (BF16, F16):
        with np.errstate(over="ignore"):
            assert eq(O.rnd(x, dt), R.round(x, dt))


@pytest.mark.parametrize("dim", (8, 64, 77, 128, 5120, 6656))
def test_rmsnorm(R, dim):
    for dt in (F64, BF16, F16):
        x = O.rnd(RNG.normal(0, 1, (7, dim)), dt)
        w = O.rnd(RNG.normal(1, 0.05, dim), dt)
        for kind in (0, 1, 2):
            assert eq(O.rmsnorm_rows(kind, x, w, 1e-6, dt), R.rmsnorm_rows(kind, x, w, 1e-6, dt))
    assert eq(O.mean_sq(x), R.mean_sq(x))
    # the f32-compat branch (f64 storage; mean_sq_f32 and the f32 chain)
    x = RNG.normal(0, 3, (7, dim))
    w = RNG.normal(1, 0.05, dim)
    for kind in (0, 1, 2):
        assert eq(O.rmsnorm_rows(kind, x, w, 1e-6, F64 | O.F32_COMPAT),
                  R.rmsnorm_rows(kind, x, w, 1e-6, F64, f32_compat=True))


@pytest.mark.parametrize("theta,dim,T", ((1e6, 128, 4096), (5e5, 128, 1024), (1e4, 256, 300)))
def test_rope(R, theta, dim, T):
    for dt in (F64, BF16, F16):
        c, s = O.rope_table(theta, dim, T, dt)
        rc, rs = R.rope_table(theta, dim, T, dt)
        assert eq(c, rc) and eq(s, rs)
        pos = RNG.integers(0, T, 16)
        x = O.rnd(RNG.normal(0, 1, (16, 1, dim)), dt)
        y = O.apply_rope(x, c, s, pos, dt)
        for t in range(16):
            assert eq(y[t, 0], R.apply_rope_vec(x[t, 0], c, s, int(pos[t]), dt))
    c, s = O.rope_table(theta, dim, T, F64 | O.F32_COMPAT)
    rc, rs = R.rope_table(theta, dim, T, F64, f32_compat=True)
    assert eq(c, rc) and eq(s, rs)


def test_output_tail(R):
    for dt in (F64, BF16, F16):
        z = O.rnd(RNG.normal(0, 30, 50000), dt)
        for mult, cap in ((1.0, 30.0), (0.7, 29.3), (3.0, 0.0)):
            assert eq(O.softcap(z, mult, cap, dt), R.output_tail(z, mult, cap, dt))
