"""GPU parity: RMSNorm rows and fused residual-add + RMSNorm vs the oracle.

Reference: muse::rmsnorm_rows (src/muse_glimmer.hpp:572-608) and the residual
loop (src/muse_glimmer.hpp:1023-1024). Gates: bitwise where the reduction order
is the reference's (dim <= 128, and every elementwise residual output); at most
1 storage ulp for bf16/f16 outputs of the tree reduction; 1e-12 relative for
f64 and 1e-6 relative for f32 against the f64 oracle.
"""
import numpy as np
import pytest

import oracle as O
from util import BF16, F16, F32, F64, from_dev, same_bits, storage, to_dev, ulp_diff16

pytestmark = pytest.mark.gpu

KINDS = (O.CENTERED, O.PLAIN, O.WEIGHTLESS)


def run_residual_norm(prims, kind, rows, dim, dt, eps=1e-6, seed=1, wmean=1.0, wstd=0.05):
    hs, h = storage(seed, (rows, dim), dt)
    xs, x = storage(seed + 1, (rows, dim), dt)
    ws, w = storage(seed + 2, (dim,), dt, wmean, wstd)
    dh, dx, dw = to_dev(hs, dt), to_dev(xs, dt), to_dev(ws, dt)
    dy = to_dev(np.zeros_like(hs), dt)
    prims.residual_rmsnorm(kind, dh, dx, None if kind == O.WEIGHTLESS else dw, eps, dy)
    y_ref, h_ref = O.residual_rmsnorm(kind, h, x, w, eps, dt)
    return from_dev(dy, dt), from_dev(dh, dt), y_ref, h_ref


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dt", (F64, BF16))
def test_config1_tiny_bitwise(prims, kind, dt):
    """Config 1: f32-drawn x, residual [16, 64], w ~ N(1, 0.1), eps 1e-6 — bitwise
    against the f64 oracle and the bf16 twin (the ordered mean_sq path)."""
    # f32-valued inputs, as the config draws them, widened to the dtype under test
    h32 = O.normal(1, (16, 64), 0.0, 1.0, F32)
    x32 = O.normal(2, (16, 64), 0.0, 1.0, F32)
    w32 = O.normal(3, (64,), 1.0, 0.1, F32)
    h, x, w = (O.rnd(O.to_f64(a, F32), dt) for a in (h32, x32, w32))
    hs, xs, ws = (O.from_f64(a, dt) for a in (h, x, w))
    dh, dx, dw = to_dev(hs, dt), to_dev(xs, dt), to_dev(ws, dt)
    dy = to_dev(np.zeros_like(hs), dt)
    prims.residual_rmsnorm(kind, dh, dx, None if kind == O.WEIGHTLESS else dw, 1e-6, dy)
    y_ref, h_ref = O.residual_rmsnorm(kind, h, x, w, 1e-6, dt)
    assert same_bits(from_dev(dh, dt), O.from_f64(h_ref, dt))
    assert same_bits(from_dev(dy, dt), O.from_f64(y_ref, dt))


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
@pytest.mark.parametrize("dim", (64, 96, 128, 13))
def test_ordered_path_bitwise(prims, dt, dim):
    """dim <= 128 runs mean_sq's exact order: bitwise in every dtype (QK-norm shape)."""
    for kind in KINDS:
        y, hn, y_ref, h_ref = run_residual_norm(prims, kind, 517, dim, dt, seed=11 + kind)
        assert same_bits(hn, O.from_f64(h_ref, dt))
        assert same_bits(y, O.from_f64(y_ref, dt)), (kind, dim)


def check_lp(y_bits, y_ref, dt, max_frac=1e-5):
    ref_bits = O.from_f64(y_ref, dt)
    d = ulp_diff16(y_bits, ref_bits)
    assert d.max() <= 1, f"max ulp {d.max()}"
    assert (d > 0).mean() <= max_frac, f"{(d > 0).sum()} of {d.size} differ by 1 ulp"
    return int((d > 0).sum())


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dim", (5120, 6656, 1000, 1032))
def test_tree_bf16_within_ulp(prims, kind, dim):
    y, hn, y_ref, h_ref = run_residual_norm(prims, kind, 193, dim, BF16, seed=21 + kind)
    assert same_bits(hn, O.from_f64(h_ref, BF16))  # the residual add is elementwise: bitwise
    check_lp(y, y_ref, BF16)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows", (257, 4096))
def test_tree_bf16_bitwise_on_exact_sums(prims, kind, rows):
    """Rows of multiples of 1/16 up to 4 in magnitude: h + x and every sum of
    squares is exact in any order, so rs is the twin's to the bit and each
    bf16 output must equal the twin's chain (f64 product, f64 -> f32 -> bf16).
    The kernel forms y in f32 first and keeps it only away from bf16 rounding
    midpoints; with random rs and w the f32 results' low halves cover the
    midpoint neighbourhood (rejected or accepted) some hundreds of times."""
    rng = np.random.default_rng(90 + kind)
    dim = 5120
    h = rng.integers(-32, 33, (rows, dim)) / 16.0
    x = rng.integers(-32, 33, (rows, dim)) / 16.0
    ws, w = storage(93 + kind, (dim,), BF16, 1.0, 0.05)
    dh, dx, dw = to_dev(O.from_f64(h, BF16), BF16), to_dev(O.from_f64(x, BF16), BF16), to_dev(ws, BF16)
    dy = to_dev(np.zeros((rows, dim), np.uint16), BF16)
    eps = 1e-6
    prims.residual_rmsnorm(kind, dh, dx, None if kind == O.WEIGHTLESS else dw, eps, dy)
    y_ref, h_ref = O.residual_rmsnorm(kind, h, x, w, eps, BF16)
    assert same_bits(from_dev(dh, BF16), O.from_f64(h_ref, BF16))
    assert same_bits(from_dev(dy, BF16), O.from_f64(y_ref, BF16))


@pytest.mark.parametrize("T", (1, 2, 3, 4, 8, 16, 32, 64))
def test_decode_shapes(prims, T):
    y, hn, y_ref, h_ref = run_residual_norm(prims, O.PLAIN, T, 5120, BF16, seed=31)
    assert same_bits(hn, O.from_f64(h_ref, BF16))
    check_lp(y, y_ref, BF16, max_frac=1e-3)


def test_f16(prims):
    y, hn, y_ref, h_ref = run_residual_norm(prims, O.CENTERED, 129, 5120, F16, seed=41, wmean=0.0, wstd=0.1)
    assert same_bits(hn, O.from_f64(h_ref, F16))
    check_lp(y, y_ref, F16)


def test_f64_within_1e12(prims):
    for kind in KINDS:
        y, hn, y_ref, h_ref = run_residual_norm(prims, kind, 64, 5120, F64, seed=51 + kind)
        assert same_bits(hn, h_ref)
        rel = np.abs(y - y_ref) / np.maximum(np.abs(y_ref), 1e-300)
        assert rel.max() <= 1e-12


def test_f32_within_1e6_of_f64_oracle(prims):
    for kind in KINDS:
        hs, h = storage(61, (64, 5120), F32)
        xs, x = storage(62, (64, 5120), F32)
        ws, w = storage(63, (5120,), F32, 1.0, 0.05)
        dh, dx, dw, dy = to_dev(hs, F32), to_dev(xs, F32), to_dev(ws, F32), to_dev(np.zeros_like(hs), F32)
        prims.residual_rmsnorm(kind, dh, dx, dw, 1e-6, dy)
        # f64 oracle on the same stream values: the residual add is the f32 materialization
        hn = O.residual_add(h, x, F32)
        y64 = O.rmsnorm_rows(kind, hn, w, 1e-6, F64)
        y = from_dev(dy, F32).astype(np.float64)
        rel = np.abs(y - y64) / np.maximum(np.abs(y64), 1e-30)
        assert rel.max() <= 1e-6


def test_plain_rmsnorm_strided_inplace(prims):
    """mg_rmsnorm_rows with a leading dimension, in place (y == x)."""
    import torch
    rows, dim, ld = 33, 5120, 5120 + 64
    xs, x = storage(71, (rows, ld), BF16)
    ws, w = storage(72, (dim,), BF16, 1.0, 0.05)
    dx = to_dev(xs, BF16)
    view = dx[:, :dim]
    prims.rmsnorm_rows(O.PLAIN, view, to_dev(ws, BF16), 1e-6, view)
    out = from_dev(dx, BF16)
    y_ref = O.rmsnorm_rows(O.PLAIN, x[:, :dim], w, 1e-6, BF16)
    check_lp(out[:, :dim], y_ref, BF16)
    assert same_bits(out[:, dim:], xs[:, dim:])  # padding untouched
    torch.cuda.synchronize()


def test_config2_full_shape(prims):
    """Config 2 at full size: bf16 [4096, 5120], w ~ N(1, 0.05), eps 1e-6."""
    y, hn, y_ref, h_ref = run_residual_norm(prims, O.PLAIN, 4096, 5120, BF16, seed=1)
    assert same_bits(hn, O.from_f64(h_ref, BF16))
    n = check_lp(y, y_ref, BF16, max_frac=1e-6)
    print(f"config2: {n} of {y.size} outputs differ from the twin by 1 ulp")


def test_deterministic(prims):
    a = run_residual_norm(prims, O.CENTERED, 300, 5120, BF16, seed=81)
    b = run_residual_norm(prims, O.CENTERED, 300, 5120, BF16, seed=81)
    assert same_bits(a[0], b[0]) and same_bits(a[1], b[1])


def test_errors(prims):
    import mgprims
    import torch
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(mgprims.MgError, match="weight is NULL"):
        prims.rmsnorm_rows(O.PLAIN, x, None, 1e-6, x)
    with pytest.raises(mgprims.MgError, match="norm kind"):
        prims.rmsnorm_rows(7, x, None, 1e-6, x)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dim", (13, 128, 5120, 6656))
def test_bf16exec_norm_rows(prims, kind, dim):
    """bf16exec's norm_rows (src/bf16exec.hpp:398-421): f32 rows, bf16 weights, bf16
    output; within 1 bf16 ulp of its f64 sequential-sum formula (the sum order differs)"""
    xs, x = storage(91 + dim, (33, dim), F32)
    ws, w = storage(92 + dim, (dim,), BF16, 1.0, 0.05)
    dy = to_dev(np.zeros((33, dim), np.uint16), BF16)
    prims.norm_rows_mixed(kind, to_dev(xs, F32), None if kind == O.WEIGHTLESS else to_dev(ws, BF16), 1e-6, dy)
    ref = O.norm_rows_mixed(kind, x, w, 1e-6, BF16)
    check_lp(from_dev(dy, BF16), ref, BF16, max_frac=1e-4)


@pytest.mark.parametrize("dtx,dtw,dty", ((BF16, F32, F32), (F16, F16, F64), (F64, BF16, F16), (F32, F32, F32)))
def test_norm_rows_mixed_formats(prims, dtx, dtw, dty):
    """other format mixes against the same formula: 16-bit outputs within 1 ulp, f32
    within 1e-6 and f64 within 1e-12 relative"""
    rows, dim = 21, 777
    xs, x = storage(95, (rows, dim), dtx)
    ws, w = storage(96, (dim,), dtw, 1.0, 0.05)
    for kind in KINDS:
        yz = np.zeros((rows, dim), np.uint16 if dty in (BF16, F16) else (np.float32 if dty == F32 else np.float64))
        dy = to_dev(yz, dty)
        prims.norm_rows_mixed(kind, to_dev(xs, dtx), to_dev(ws, dtw), 1e-6, dy)
        ref = O.norm_rows_mixed(kind, x, w, 1e-6, dty)
        got = from_dev(dy, dty)
        if dty in (BF16, F16):
            check_lp(got, ref, dty, max_frac=1e-3)
        else:
            rel = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)
            assert rel.max() <= (1e-6 if dty == F32 else 1e-12)


def test_norm_rows_mixed_strided_inplace(prims):
    rows, dim, ld = 9, 640, 700
    xs, x = storage(97, (rows, ld), F32)
    ws, w = storage(98, (dim,), F32, 1.0, 0.05)
    dx = to_dev(xs, F32)
    view = dx[:, :dim]
    prims.norm_rows_mixed(O.PLAIN, view, to_dev(ws, F32), 1e-6, view)
    out = from_dev(dx, F32)
    ref = O.norm_rows_mixed(O.PLAIN, np.ascontiguousarray(x[:, :dim]), w, 1e-6, F32)
    rel = np.abs(out[:, :dim].astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= 1e-6
    assert same_bits(out[:, dim:], xs[:, dim:])


# --------------------------------------- norm_rows_f32: the embedding norm
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dim", (5120, 6656))
def test_norm_rows_f32_in_place(prims, kind, dim):
    """bf16exec's norm_rows_f32 (src/bf16exec.hpp:422-442; the GPU engine's k_rmsnorm_f32,
    src/gpu/gpu_engine.cpp:392-415) as mg_norm_rows_mixed with y = MG_BF16_AS_F32, in place
    on f32 rows of N(0,1): every stored word is a bf16 value, within 1 bf16 ulp of the
    oracle's restatement (pinned bitwise to the compiled reference), and a Centered call
    is weight-less as in the reference"""
    xs, x = storage(101 + dim, (65, dim), F32)
    ws, w = storage(102 + dim, (dim,), BF16, 1.0, 0.05)
    dx = to_dev(xs, F32)
    prims.norm_rows_mixed(kind, dx, None if kind == O.WEIGHTLESS else to_dev(ws, BF16), 1e-6, dx, bf16_as_f32=True)
    got = from_dev(dx, F32).view(np.uint32)
    assert ((got & 0xffff) == 0).all()
    ref = O.norm_rows_f32(kind, x, w, 1e-6)
    check_lp((got >> 16).astype(np.uint16), ref, BF16, max_frac=1e-3)


@pytest.mark.parametrize("kind", KINDS)
def test_norm_rows_f32_bitwise_on_exact_sums(prims, kind):
    """f32 rows of multiples of 1/16: every sum of squares is exact in any order, so the
    device's bf16-in-f32 outputs equal the reference's sequential-sum chain bit for bit"""
    rng = np.random.default_rng(110 + kind)
    rows, dim = 257, 6656
    x = rng.integers(-32, 33, (rows, dim)) / 16.0
    ws, w = storage(111 + kind, (dim,), BF16, 1.0, 0.05)
    dx = to_dev(x.astype(np.float32), F32)
    dy = to_dev(np.zeros((rows, dim), np.float32), F32)
    prims.norm_rows_mixed(kind, dx, None if kind == O.WEIGHTLESS else to_dev(ws, BF16), 1e-6, dy, bf16_as_f32=True)
    ref = O.norm_rows_f32(kind, x, w, 1e-6)
    assert same_bits(from_dev(dy, F32), ref.astype(np.float32))


def test_norm_rows_f32_reference_golden(prims):
    """the reference's own norm_rows_f32 outputs (tests/golden/bf16exec.npz): within 1 bf16 ulp"""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "bf16exec.npz"))
    for dim in (13, 640, 6656):
        for kind in KINDS:
            dx = to_dev(g[f"x{dim}"], F32)
            dw = None if kind == O.WEIGHTLESS else to_dev(g[f"w{dim}"], BF16)
            prims.norm_rows_mixed(kind, dx, dw, 1e-6, dx, bf16_as_f32=True)
            got = (from_dev(dx, F32).view(np.uint32) >> 16).astype(np.uint16)
            want = (g[f"f{dim}_k{kind}"].view(np.uint32) >> 16).astype(np.uint16)
            assert ulp_diff16(got, want).max() <= 1, (dim, kind)
