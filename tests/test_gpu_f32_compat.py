"""GPU parity: the --hf-f32-compat chains and the f64 softmax.

Reference: the f64 run with --hf-f32-compat (src/main.cpp:164-165;
src/muse_glimmer.hpp:951-955) places stock HF's f32 upcasts:
  rmsnorm_rows' f32 branch with mean_sq_f32 (530-556, 581-594), also as the
  QK-norm (799-803); build_rope_table's f32 chain stored as double(float(v))
  (634-657); the f32 softmax of attention_forward (856-870).
All three are bitwise against the oracle, which matches the compiled reference
bit for bit (tests/test_oracle_ref.py, the golden fixtures) and, for the
softmax, its known answers (tests/test_oracle_math.py). The pure f64 softmax
sums in a fixed parallel order: within 1e-12 relative of the f64 oracle.
"""
import os

import numpy as np
import pytest

import oracle as O
from util import F64, from_dev, same_bits, to_dev

pytestmark = pytest.mark.gpu
C64 = F64 | O.F32_COMPAT
KINDS = (O.CENTERED, O.PLAIN, O.WEIGHTLESS)
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f64(seed, shape, mean=0.0, std=1.0):
    return O.to_f64(O.normal(seed, shape, mean, std, F64), F64)


@pytest.mark.parametrize("dim", (13, 64, 128, 640, 5120))
def test_rmsnorm_compat_bitwise(prims, dim):
    x = f64(200 + dim, (37, dim), 0.0, 2.0)
    w = f64(300 + dim, (dim,), 1.0, 0.05)
    for kind in KINDS:
        dx, dy = to_dev(x, F64), to_dev(np.zeros_like(x), F64)
        prims.rmsnorm_rows(kind, dx, None if kind == O.WEIGHTLESS else to_dev(w, F64), 1e-6, dy, f32_compat=True)
        ref = O.rmsnorm_rows(kind, x, w, 1e-6, C64)
        assert same_bits(from_dev(dy, F64), ref), (kind, dim)


@pytest.mark.parametrize("dim", (64, 77, 5120))
def test_residual_rmsnorm_compat_bitwise(prims, dim):
    """h = h + x in f64 (the twin's f64 residual), then the f32 chain."""
    h, x = f64(401, (29, dim)), f64(402, (29, dim))
    w = f64(403, (dim,), 1.0, 0.05)
    for kind in KINDS:
        dh, dx, dy = to_dev(h, F64), to_dev(x, F64), to_dev(np.zeros_like(h), F64)
        prims.residual_rmsnorm(kind, dh, dx, None if kind == O.WEIGHTLESS else to_dev(w, F64), 1e-6, dy,
                               f32_compat=True)
        y_ref, h_ref = O.residual_rmsnorm(kind, h, x, w, 1e-6, C64)
        assert same_bits(from_dev(dh, F64), h_ref)
        assert same_bits(from_dev(dy, F64), y_ref), (kind, dim)


def test_rmsnorm_compat_strided_inplace(prims):
    rows, dim, ld = 21, 640, 700
    x = f64(410, (rows, ld))
    w = f64(411, (dim,), 1.0, 0.05)
    dx = to_dev(x, F64)
    view = dx[:, :dim]
    prims.rmsnorm_rows(O.CENTERED, view, to_dev(w, F64), 1e-6, view, f32_compat=True)
    out = from_dev(dx, F64)
    assert same_bits(out[:, :dim], O.rmsnorm_rows(O.CENTERED, np.ascontiguousarray(x[:, :dim]), w, 1e-6, C64))
    assert same_bits(out[:, dim:], x[:, dim:])


def test_norms_golden_compat(prims):
    """the reference's own outputs (tests/golden/norms.npz, compiled reference)"""
    g = np.load(os.path.join(GOLDEN, "norms.npz"))
    for dim in (13, 128, 640):
        x, w = g[f"x{dim}"], g[f"w{dim}"]
        for kind in KINDS:
            dy = to_dev(np.zeros_like(x), F64)
            prims.rmsnorm_rows(kind, to_dev(x, F64), None if kind == O.WEIGHTLESS else to_dev(w, F64), 1e-6, dy,
                               f32_compat=True)
            assert same_bits(from_dev(dy, F64), g[f"y{dim}_k{kind}_compat"]), (dim, kind)


@pytest.mark.parametrize("theta,dim,T", ((1e6, 128, 64), (5e5, 128, 48), (1e4, 64, 40)))
def test_rope_table_golden_compat(prims, theta, dim, T):
    import torch
    g = np.load(os.path.join(GOLDEN, "rope.npz"))
    tag = f"{int(theta)}_{dim}"
    co, si = prims.build_rope_table(theta, dim, T, torch.float64, f32_compat=True)
    assert same_bits(co.cpu().numpy(), g[f"cos_{tag}_compat"])
    assert same_bits(si.cpu().numpy(), g[f"sin_{tag}_compat"])


def test_rope_table_compat_config3(prims):
    import torch
    co, si = prims.build_rope_table(1e6, 128, 4096, torch.float64, f32_compat=True)
    c, s = O.rope_table(1e6, 128, 4096, C64)
    assert same_bits(co.cpu().numpy(), c) and same_bits(si.cpu().numpy(), s)


def test_qk_norm_rope_compat(prims):
    """the compat QK path: f32-chain QK-norm, f64 scale, f64 RoPE over the compat
    table, cache append; equal to the separate oracle steps bit for bit"""
    import torch
    T, qh, kh, D, slots = 19, 8, 2, 128, 32
    q, k, v = f64(420, (T, qh, D), 0, 2), f64(421, (T, kh, D), 0, 2), f64(422, (T, kh, D))
    c, s = O.rope_table(1e6, D, T, C64)
    dq, dk, dv = to_dev(q, F64), to_dev(k, F64), to_dev(v, F64)
    kc = torch.zeros((slots, kh, D), dtype=torch.float64, device="cuda:0")
    vc = torch.zeros_like(kc)
    prims.qk_norm_rope(dq, dk, 1e-6, 3.87, to_dev(c, F64), to_dev(s, F64), v=dv, k_cache=kc, v_cache=vc,
                       f32_compat=True)
    rq = O.rmsnorm_rows(O.WEIGHTLESS, q.reshape(-1, D), None, 1e-6, C64).reshape(q.shape)
    rk = O.rmsnorm_rows(O.WEIGHTLESS, k.reshape(-1, D), None, 1e-6, C64).reshape(k.shape)
    rq = O.scale(rq, 3.87, F64)
    pos = np.arange(T)
    rq, rk = O.apply_rope(rq, c, s, pos, F64), O.apply_rope(rk, c, s, pos, F64)
    assert same_bits(from_dev(dq, F64), rq)
    assert same_bits(from_dev(dk, F64), rk)
    kcn = kc.cpu().numpy()
    assert same_bits(kcn[:T], rk) and same_bits(vc.cpu().numpy()[:T], v)


def run_sm(prims, x, scale, mask, window, q0, compat, softcap=0.0):
    dx = to_dev(x, F64)
    dy = to_dev(np.full_like(x, 7.0), F64)
    prims.softmax_rows(dx, dy, scale, mask, window, q0, softcap, f32_compat=compat)
    ref = O.softmax_rows(x, scale, mask, window, q0, softcap, C64 if compat else F64, F64)
    return from_dev(dy, F64), ref


@pytest.mark.parametrize("mask,window,q0", ((O.MASK_NONE, 0, 0), (O.MASK_CAUSAL, 0, 0), (O.MASK_CAUSAL, 0, 300),
                                            (O.MASK_WINDOW, 64, 100), (O.MASK_BIWINDOW, 20, 50)))
def test_softmax_compat_bitwise(prims, mask, window, q0):
    x = f64(430 + mask, (3, 70, 333), 0.0, 20.0)
    y, ref = run_sm(prims, x, 0.088, mask, window, q0, True)
    assert same_bits(y, ref)


def test_softmax_compat_long_rows(prims):
    """decode rows (q = 1) over 131072 keys, and ragged lengths around the
    64-key steps of the ascending chain"""
    x = f64(440, (4, 1, 131072), 0.0, 3.0)
    y, ref = run_sm(prims, x, 1.0, O.MASK_CAUSAL, 0, 131071 - 17, True)
    assert same_bits(y, ref)
    for kc in (1, 63, 64, 65, 129, 4097):
        x = f64(441 + kc, (2, 3, kc), 0.0, 5.0)
        y, ref = run_sm(prims, x, 0.5, O.MASK_NONE, 0, 0, True)
        assert same_bits(y, ref), kc


def test_softmax_compat_known_answer(prims):
    """sum32 stays exactly 1 on [0, s, ..., s] with float(exp(s)) just below
    2^-24 (the ascending f32 chain; see tests/test_oracle_math.py)"""
    s32 = np.float32(-24 * np.log(2.0))
    while O.exp(np.array([float(s32)]))[0].astype(np.float32) >= np.float32(2.0 ** -24):
        s32 = np.nextafter(s32, np.float32(-np.inf))
    row = np.full((1, 1, 1001), float(s32))
    row[0, 0, 0] = 0.0
    y, ref = run_sm(prims, row, 1.0, O.MASK_NONE, 0, 0, True)
    assert y[0, 0, 0] == 1.0 and same_bits(y, ref)


def test_softmax_compat_nonfinite(prims):
    x = f64(450, (1, 6, 200), 0.0, 4.0)
    x[0, 0, 5] = np.nan
    x[0, 1, 7] = np.inf
    x[0, 2, :] = -np.inf
    x[0, 3, 9] = -np.inf
    y, ref = run_sm(prims, x, 1.0, O.MASK_NONE, 0, 0, True)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert same_bits(y[ok], ref[ok])


@pytest.mark.parametrize("cap", (0.0, 30.0))
def test_softmax_f64_within_1e12(prims, cap):
    x = f64(460, (5, 40, 3000), 0.0, 30.0)
    y, ref = run_sm(prims, x, 0.088, O.MASK_CAUSAL, 0, 2980, False, cap)
    assert np.all((y == 0.0) == (ref == 0.0))
    nz = ref != 0.0
    assert np.abs(y[nz] / ref[nz] - 1).max() <= 1e-12
    x = f64(461, (2, 1, 131072), 0.0, 3.0)
    y, ref = run_sm(prims, x, 1.0, O.MASK_WINDOW, 4096, 131071, False)
    nz = ref != 0.0
    assert np.all(y[~nz] == 0.0) and np.abs(y[nz] / ref[nz] - 1).max() <= 1e-12


def test_errors(prims):
    import torch
    xb = torch.zeros((4, 64), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(Exception, match="f64 storage only"):
        prims.rmsnorm_rows(O.WEIGHTLESS, xb, None, 1e-6, xb, f32_compat=True)
    x = torch.zeros((1, 2, 64), dtype=torch.float64, device="cuda:0")
    with pytest.raises(Exception, match="no softcap"):
        prims.softmax_rows(x, x, 1.0, softcap=30.0, f32_compat=True)
    y = torch.zeros((1, 2, 64), dtype=torch.float32, device="cuda:0")
    with pytest.raises(Exception, match="f64 probabilities"):
        prims.softmax_rows(x, y, 1.0)
    with pytest.raises(Exception, match="unknown dtype"):
        prims.build_rope_table(1e6, 128, 16, torch.float32, f32_compat=True)
