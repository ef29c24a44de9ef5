"""GPU parity: SwiGLU, sigmoid output gate, residual add, qk scale, output tail.

Reference loops: SwiGLU src/muse_glimmer.hpp:1036-1039, output gate 896-906,
residual 1023-1024, qk scale 803-807, apply_output_tail 920-943. All are
elementwise, so the gate is bitwise against the oracle (the twin in bf16/f16,
f32 materializations for f32, the pure form for f64), including exhaustively
over every 16-bit gate input.
"""
import numpy as np
import pytest

import oracle as O
from util import BF16, F16, F32, F64, from_dev, same_bits, same_bits_or_nan, storage, to_dev

pytestmark = pytest.mark.gpu


def all16(dt):
    """every 16-bit pattern as storage bits and values (NaN patterns included)"""
    bits = np.arange(65536, dtype=np.uint16)
    return bits, O.to_f64(bits, dt)


def mismatches(a, b, *cols, n=12):
    """first differing positions with the values that produced them"""
    idx = np.nonzero(a != b)[0][:n]
    return [(int(i), int(a[i]), int(b[i]), *(float(c[i]) for c in cols)) for i in idx]


@pytest.mark.parametrize("dt", (BF16, F16))
@pytest.mark.parametrize("gate", (False, True))
@pytest.mark.parametrize("unit", (1.0, -1.0))
def test_table_contents(prims, dt, gate, unit):
    """with the other operand = +-1 the output is +-rnd(f(g)) itself: every table
    entry against the twin's rnd(silu(g)) / rnd(sigmoid(g))"""
    gb, g = all16(dt)
    one = np.full(65536, unit)
    dg, d1 = to_dev(gb, dt), to_dev(O.from_f64(one, dt), dt)
    dout = to_dev(np.zeros(65536, np.uint16), dt)
    if gate:
        prims.sigmoid_gate(d1, dg, dout)
        ref = O.sigmoid_gate(one, g, dt)
    else:
        prims.swiglu(dg, d1, dout)
        ref = O.swiglu(g, one, dt)
    out, rb = from_dev(dout, dt), O.from_f64(ref, dt)
    assert same_bits_or_nan(out, rb, dt), mismatches(out, rb, g)


@pytest.mark.parametrize("dt", (BF16, F16))
@pytest.mark.parametrize("gate", (False, True))
def test_exhaustive_16bit_gate_inputs(prims, dt, gate):
    """Every 16-bit gate value x a random up/pv operand: bitwise vs the twin."""
    gb, g = all16(dt)
    us, u = storage(5, (65536,), dt)
    dg, du = to_dev(gb, dt), to_dev(us, dt)
    dout = to_dev(np.zeros(65536, np.uint16), dt)
    if gate:
        prims.sigmoid_gate(du, dg, dout)
        ref = O.sigmoid_gate(u, g, dt)
    else:
        prims.swiglu(dg, du, dout)
        ref = O.swiglu(g, u, dt)
    out, rb = from_dev(dout, dt), O.from_f64(ref, dt)
    assert same_bits_or_nan(out, rb, dt), mismatches(out, rb, g, u)


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
@pytest.mark.parametrize("gate", (False, True))
@pytest.mark.parametrize("n", (64 * 25600 + 5, 33 * 19968, 1000, 7))
def test_gate_random(prims, dt, gate, n):
    gs, g = storage(4, (n,), dt)
    us, u = storage(5, (n,), dt)
    dg, du = to_dev(gs, dt), to_dev(us, dt)
    dout = to_dev(np.zeros_like(gs), dt)
    if gate:
        prims.sigmoid_gate(du, dg, dout)
        ref = O.sigmoid_gate(u, g, dt)
    else:
        prims.swiglu(dg, du, dout)
        ref = O.swiglu(g, u, dt)
    assert same_bits(from_dev(dout, dt), O.from_f64(ref, dt))


def test_swiglu_unaligned(prims):
    """operands that are not 16-byte aligned take the scalar table kernel"""
    n = 10001
    gs, g = storage(6, (n + 1,), BF16)
    us, u = storage(7, (n + 1,), BF16)
    dg, du = to_dev(gs, BF16), to_dev(us, BF16)
    dout = to_dev(np.zeros(n + 1, np.uint16), BF16)
    prims.swiglu(dg[1:], du[1:], dout[1:])
    ref = O.swiglu(g[1:], u[1:], BF16)
    assert same_bits(from_dev(dout, BF16)[1:], O.from_f64(ref, BF16))


def test_swiglu_config3_full(prims):
    """Config 3 SwiGLU at full size: bf16 gate/up [4096, 25600] ~ N(0, 1)."""
    shape = (4096, 25600)
    gs, g = storage(4, shape, BF16)
    us, u = storage(5, shape, BF16)
    dg, du = to_dev(gs, BF16), to_dev(us, BF16)
    dout = to_dev(np.zeros_like(gs), BF16)
    prims.swiglu(dg, du, dout)
    assert same_bits(from_dev(dout, BF16), O.from_f64(O.swiglu(g, u, BF16), BF16))


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
def test_residual_add(prims, dt):
    n = 4096 * 33 + 3
    hs, h = storage(8, (n,), dt)
    xs, x = storage(9, (n,), dt, 0.0, 3.0)
    dh, dx = to_dev(hs, dt), to_dev(xs, dt)
    prims.residual_add(dh, dx)
    assert same_bits(from_dev(dh, dt), O.from_f64(O.residual_add(h, x, dt), dt))


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
def test_qk_scale(prims, dt):
    n = 40 * 128 * 97 + 1
    xs, x = storage(10, (n,), dt)
    dx = to_dev(xs, dt)
    prims.scale(dx, 3.87)
    assert same_bits(from_dev(dx, dt), O.from_f64(O.scale(x, 3.87, dt), dt))


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
@pytest.mark.parametrize("mult,cap", ((1.0, 30.0), (0.5, 30.0), (2.0, 0.0), (1.0, 0.0)))
def test_output_tail(prims, dt, mult, cap):
    n = 201088 + 17
    zs, z = storage(11, (n,), dt, 0.0, 40.0 if dt != F16 else 20.0)
    dz = to_dev(zs, dt)
    prims.apply_output_tail(dz, mult, cap)
    assert same_bits(from_dev(dz, dt), O.from_f64(O.softcap(z, mult, cap, dt), dt))


def test_output_tail_exhaustive_bf16(prims):
    gb, g = all16(BF16)
    dz = to_dev(gb.copy(), BF16)
    prims.apply_output_tail(dz, 1.0, 30.0)
    out = from_dev(dz, BF16)
    ref = O.from_f64(O.softcap(g, 1.0, 30.0, BF16), BF16)
    assert same_bits_or_nan(out, ref, BF16)


def test_errors(prims):
    import mgprims
    import torch
    x = torch.zeros(16, dtype=torch.int32, device="cuda:0")
    with pytest.raises(KeyError):
        prims.swiglu(x, x, x)  # not a storage dtype the ABI knows
    a = torch.zeros(16, dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(mgprims.MgError, match="aligned"):
        prims.residual_add(a[1:], a[1:])
