"""CPU: the oracle restatement against the golden fixtures written by the
reference's own compiled code (tests/golden/make_golden.py). Every comparison
is bitwise."""
import os

import numpy as np
import pytest

import oracle as O
from util import same_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F64, BF16, F16, F32 = O.F64, O.BF16, O.F16, O.F32


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def eq(a, b):
    """bitwise, NaN payloads included"""
    return same_bits(np.asarray(a, np.float64), np.asarray(b, np.float64))


def test_rounding():
    g = load("rounding.npz")
    assert eq(O.rnd(g["x"], BF16), g["bf16"])
    assert eq(O.rnd(g["x"], F16), g["f16"])
    dec = O.to_f64(np.arange(65536, dtype=np.uint16), F16)
    nan = np.isnan(g["f16_decode"])
    assert np.array_equal(np.isnan(dec), nan)
    assert eq(dec[~nan], g["f16_decode"][~nan])


def test_fmath():
    g = load("fmath.npz")
    assert eq(O.exp(g["x"]), g["exp"])
    assert eq(O.silu(g["x"]), g["silu"])
    assert eq(O.sigmoid(g["x"]), g["sigmoid"])
    assert eq(O.tanh(g["xt"]), g["tanh"])
    assert eq(O.sin(g["xs"]), g["sin"])
    assert eq(O.cos(g["xs"]), g["cos"])
    for base, key in ((1e6, "pow_1e6"), (5e5, "pow_5e5"), (1e4, "pow_1e4")):
        assert eq(O.pow_(base, g["pow_e"]), g[key])


@pytest.mark.parametrize("dt,tag", ((F64, "f64"), (BF16, "bf16")))
def test_config1(dt, tag):
    g = load("config1.npz")
    x, r, w = (O.rnd(g[k], dt) for k in ("x", "residual", "w"))
    for kind, kn in ((O.CENTERED, "centered"), (O.PLAIN, "plain"), (O.WEIGHTLESS, "weightless")):
        y, h = O.residual_rmsnorm(kind, x, r, w, 1e-6, dt)
        assert eq(h, g[f"{tag}_h"])
        assert eq(y, g[f"{tag}_{kn}_y"])
    gate, up = O.rnd(g["gate"], dt), O.rnd(g["up"], dt)
    assert eq(O.swiglu(gate, up, dt), g[f"{tag}_swiglu"])


@pytest.mark.parametrize("dim", (13, 128, 640))
def test_norms(dim):
    g = load("norms.npz")
    for dt in (F64, BF16, F16):
        x, w = O.rnd(g[f"x{dim}"], dt), O.rnd(g[f"w{dim}"], dt)
        for kind in (0, 1, 2):
            assert eq(O.rmsnorm_rows(kind, x, w, 1e-6, dt), g[f"y{dim}_k{kind}_d{dt}"])
    for kind in (0, 1, 2):
        assert eq(O.rmsnorm_rows(kind, g[f"x{dim}"], g[f"w{dim}"], 1e-6, F64 | O.F32_COMPAT),
                  g[f"y{dim}_k{kind}_compat"])


@pytest.mark.parametrize("theta,dim,T", ((1e6, 128, 64), (5e5, 128, 48), (1e4, 64, 40)))
def test_rope(theta, dim, T):
    g = load("rope.npz")
    tag = f"{int(theta)}_{dim}"
    for dt in (F64, BF16, F16):
        c, s = O.rope_table(theta, dim, T, dt)
        assert eq(c, g[f"cos_{tag}_d{dt}"]) and eq(s, g[f"sin_{tag}_d{dt}"])
        x = g[f"x_{tag}_d{dt}"]
        rot = O.apply_rope(x[:, None, :], c, s, np.arange(T), dt)[:, 0, :]
        assert eq(rot, g[f"rot_{tag}_d{dt}"])
    c, s = O.rope_table(theta, dim, T, F64 | O.F32_COMPAT)
    assert eq(c, g[f"cos_{tag}_compat"]) and eq(s, g[f"sin_{tag}_compat"])


def test_output_tail():
    g = load("tail.npz")
    for dt in (F64, BF16, F16):
        z = g[f"z_d{dt}"]
        for mult, cap in ((1.0, 30.0), (0.5, 30.0), (2.0, 0.0)):
            assert eq(O.softcap(z, mult, cap, dt), g[f"tail_d{dt}_m{mult}_c{cap}"])


def test_bf16exec_norms():
    """bf16exec's norm_rows (bf16 out) and norm_rows_f32 (bf16 values kept in f32, weight
    for Plain only), both compiled from src/bf16exec.hpp, against the oracle's
    or_norm_rows_mixed and or_norm_rows_f32: bitwise at every kind and dim 13 / 640 / 6656"""
    g = load("bf16exec.npz")
    for dim in (13, 640, 6656):
        x = g[f"x{dim}"].astype(np.float64)
        w = O.to_f64(g[f"w{dim}"], BF16)
        for kind in (0, 1, 2):
            wk = None if kind == 2 else w
            assert eq(O.norm_rows_f32(kind, x, wk, 1e-6), g[f"f{dim}_k{kind}"])
            assert np.array_equal(O.from_f64(O.norm_rows_mixed(kind, x, wk, 1e-6, BF16), BF16), g[f"y{dim}_k{kind}"])
    # the reference's rule: norm_rows_f32 applies the weight for Plain only, so its
    # Centered output is the weight-less one (src/bf16exec.hpp:437-438)
    assert eq(g["f640_k0"], g["f640_k2"]) and not eq(g["f640_k1"], g["f640_k2"])
