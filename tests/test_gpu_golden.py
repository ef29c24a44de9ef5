"""GPU parity against the golden fixtures written by the reference's own
compiled code (tests/golden/make_golden.py): configs[0] (residual-add +
RMSNorm and SwiGLU on the tiny shapes, f64 and bf16 twin), the RoPE tables and
rotations, and the output tail — all bitwise, through the C ABI."""
import os

import numpy as np
import pytest

import oracle as O
from util import BF16, F16, F64, from_dev, same_bits, to_dev, torch_dtype

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.mark.parametrize("dt,tag", ((F64, "f64"), (BF16, "bf16")))
def test_config1(prims, dt, tag):
    g = load("config1.npz")
    x, r, w = (O.from_f64(O.rnd(g[k], dt), dt) for k in ("x", "residual", "w"))
    for kind, kn in ((O.CENTERED, "centered"), (O.PLAIN, "plain"), (O.WEIGHTLESS, "weightless")):
        dh, dx, dw = to_dev(x, dt), to_dev(r, dt), to_dev(w, dt)
        dy = to_dev(np.zeros_like(x), dt)
        prims.residual_rmsnorm(kind, dh, dx, dw, 1e-6, dy)
        assert same_bits(from_dev(dh, dt), O.from_f64(g[f"{tag}_h"], dt))
        assert same_bits(from_dev(dy, dt), O.from_f64(g[f"{tag}_{kn}_y"], dt)), kn
    gate, up = (O.from_f64(O.rnd(g[k], dt), dt) for k in ("gate", "up"))
    dout = to_dev(np.zeros_like(gate), dt)
    prims.swiglu(to_dev(gate, dt), to_dev(up, dt), dout)
    assert same_bits(from_dev(dout, dt), O.from_f64(g[f"{tag}_swiglu"], dt))


@pytest.mark.parametrize("theta,dim,T", ((1e6, 128, 64), (5e5, 128, 48), (1e4, 64, 40)))
def test_rope(prims, theta, dim, T):
    g = load("rope.npz")
    tag = f"{int(theta)}_{dim}"
    for dt in (F64, BF16, F16):
        co, si = prims.build_rope_table(theta, dim, T, torch_dtype(dt))
        assert same_bits(from_dev(co, dt), O.from_f64(g[f"cos_{tag}_d{dt}"], dt))
        assert same_bits(from_dev(si, dt), O.from_f64(g[f"sin_{tag}_d{dt}"], dt))
        x = to_dev(O.from_f64(g[f"x_{tag}_d{dt}"], dt), dt).reshape(T, 1, dim)
        prims.apply_rope(x, None, co, si)
        assert same_bits(from_dev(x, dt).reshape(T, dim), O.from_f64(g[f"rot_{tag}_d{dt}"], dt))


def test_output_tail(prims):
    g = load("tail.npz")
    for dt in (F64, BF16, F16):
        for mult, cap in ((1.0, 30.0), (0.5, 30.0), (2.0, 0.0)):
            z = to_dev(O.from_f64(g[f"z_d{dt}"], dt), dt)
            prims.apply_output_tail(z, mult, cap)
            assert same_bits(from_dev(z, dt), O.from_f64(g[f"tail_d{dt}_m{mult}_c{cap}"], dt))


@pytest.mark.parametrize("dim", (13, 128, 640))
def test_norms(prims, dim):
    g = load("norms.npz")
    for dt in (F64, BF16, F16):
        x = O.from_f64(O.rnd(g[f"x{dim}"], dt), dt)
        w = O.from_f64(O.rnd(g[f"w{dim}"], dt), dt)
        for kind in (0, 1, 2):
            dy = to_dev(np.zeros_like(x), dt)
            prims.rmsnorm_rows(kind, to_dev(x, dt), None if kind == 2 else to_dev(w, dt), 1e-6, dy)
            out, ref = from_dev(dy, dt), O.from_f64(g[f"y{dim}_k{kind}_d{dt}"], dt)
            if dim <= 128:
                assert same_bits(out, ref)  # the reference's mean_sq order
            elif dt == F64:
                assert np.abs(out / ref - 1).max() <= 1e-12
            else:
                d = np.abs(out.astype(np.int32) - ref.astype(np.int32))
                assert d.max() <= 1
