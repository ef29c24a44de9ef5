"""GPU parity: fused QK-norm + qk-scale + RoPE + KV-cache append.

Reference: the sequence of src/muse_glimmer.hpp:799-819 (weight-less
rmsnorm_rows over head_dim for q and k, q *= qk_scale, apply_rope over
(t, head)) and the cache append of k_kv_append (src/gpu/gpu_engine.cpp:481-492,
slot = position % slots). The oracle runs the same steps one after another;
the fused kernel must match it bit for bit in every dtype.
"""
import numpy as np
import pytest

import oracle as O
from util import BF16, F16, F32, F64, from_dev, same_bits, same_bits_or_nan, storage, to_dev

pytestmark = pytest.mark.gpu

EPS = 1e-6
QK = 3.87


def oracle_seq(q, k, dt, theta, dim, table_T, pos, use_rope):
    T, qh, _ = q.shape
    kh = k.shape[1]
    rq = O.rmsnorm_rows(O.WEIGHTLESS, q.reshape(T * qh, dim), None, EPS, dt).reshape(q.shape)
    rk = O.rmsnorm_rows(O.WEIGHTLESS, k.reshape(T * kh, dim), None, EPS, dt).reshape(k.shape)
    rq = O.scale(rq, QK, dt)
    if use_rope:
        rc, rs = O.rope_table(theta, dim, table_T, dt)
        rq = O.apply_rope(rq, rc, rs, pos, dt)
        rk = O.apply_rope(rk, rc, rs, pos, dt)
    return rq, rk


def run_case(prims, dt, T, qh, kh, dim, theta=1e6, pos0=0, positions=None, table_T=None, use_rope=True,
             slots=0, with_v=True, specials=False):
    import torch
    table_T = table_T or (pos0 + T)
    qs, q = storage(31, (T, qh, dim), dt)
    ks, k = storage(32, (T, kh, dim), dt)
    if specials:
        big = 1e30 if dt == BF16 else 6e4
        q[0, 0, 5] = np.nan           # a NaN row: rs and every output NaN
        q[1, 3, :] = 0.0              # an all-zero row: rs = 1/sqrt(eps), outputs +-0
        q[1, 3, 9] = -0.0
        q[2, 2, 7] = np.inf           # inf: mean_sq inf, rs 0, inf * 0 = NaN
        q[3, 0, :] *= big             # large values: mean_sq near the top of the range
        k[0, 1, 3] = -np.inf
        k[2, 0, 64:] = 0.0            # the rotated half zero
        qs, q = O.from_f64(q, dt), O.to_f64(O.from_f64(q, dt), dt)
        ks, k = O.from_f64(k, dt), O.to_f64(O.from_f64(k, dt), dt)
    vs, v = storage(33, (T, kh, dim), dt)
    dq, dk, dv = to_dev(qs, dt), to_dev(ks, dt), to_dev(vs, dt)
    dco = dsi = None
    if use_rope:
        rc, rs = O.rope_table(theta, dim, table_T, dt)
        dco, dsi = to_dev(O.from_f64(rc, dt), dt), to_dev(O.from_f64(rs, dt), dt)
    dpos = None
    if positions is not None:
        pos = np.asarray(positions, np.int64)
        dpos = torch.from_numpy(pos).to("cuda:0")
    else:
        pos = np.arange(pos0, pos0 + T, dtype=np.int64)
    kc = vc = None
    cache0 = None
    if slots:
        cache0 = O.from_f64(np.full((slots, kh, dim), 0.25), dt)
        kc, vc = to_dev(cache0, dt), to_dev(cache0, dt)
        if not with_v:
            vc = None
    prims.qk_norm_rope(dq, dk, EPS, QK, dco, dsi, dpos, pos0, dv if with_v else None, kc, vc)
    rq, rk = oracle_seq(q, k, dt, theta, dim, table_T, pos, use_rope)
    if specials and dt != BF16:  # bf16's NaN is the one pattern 0x7FC0: bitwise there
        assert same_bits_or_nan(from_dev(dq, dt), O.from_f64(rq, dt), dt)
        assert same_bits_or_nan(from_dev(dk, dt), O.from_f64(rk, dt), dt)
        return
    assert same_bits(from_dev(dq, dt), O.from_f64(rq, dt))
    assert same_bits(from_dev(dk, dt), O.from_f64(rk, dt))
    if slots:
        ek = O.to_f64(cache0, dt).copy()
        ev = O.to_f64(cache0, dt).copy()
        for t in range(T):  # later tokens overwrite earlier ones in the ring, as sequential appends do
            if pos[t] >= 0:
                ek[pos[t] % slots] = rk[t]
                ev[pos[t] % slots] = v[t]
        assert same_bits(from_dev(kc, dt), O.from_f64(ek, dt))
        if with_v:
            assert same_bits(from_dev(vc, dt), O.from_f64(ev, dt))


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
def test_sequence_bitwise(prims, dt):
    run_case(prims, dt, 65, 40, 8, 128, pos0=7, slots=128)


@pytest.mark.parametrize("dt", (BF16, F16))
def test_special_values(prims, dt):
    """NaN, inf, zero and large rows through the fused sequence (16-bit paths;
    NaN has to meet NaN, its sign being unspecified by IEEE)"""
    run_case(prims, dt, 8, 40, 8, 128, pos0=3, specials=True)


def test_prefill_shape_bf16(prims):
    """config-3 shapes: q [4096, 40, 128], k [4096, 8, 128], theta 1e6, positions 0..4095"""
    run_case(prims, BF16, 4096, 40, 8, 128, slots=4096)


def test_nope_layer_and_no_cache(prims):
    run_case(prims, BF16, 33, 40, 8, 128, use_rope=False)


def test_positions_array_ring_wrap(prims):
    """explicit positions wrapping a ring of 16 slots (distinct slots: two
    tokens of one call on one slot would race, as in the reference), no v"""
    pos = [3, 40, 17, 1002, 2, 31, 604, 5]
    run_case(prims, BF16, len(pos), 32, 4, 128, theta=5e5, positions=pos, table_T=2048, slots=16,
             with_v=False)


def test_odd_shapes(prims):
    """head_dim 64 (theta 1e4), one kv head, a single token"""
    run_case(prims, BF16, 1, 3, 1, 64, theta=1e4, pos0=99, slots=8)
    run_case(prims, F32, 5, 2, 2, 18, theta=1e4, pos0=3, slots=7)  # half = 9, scalar staging


def wide_rows(seed, shape, dt, span):
    """values +-m * 2^e with e drawn over `span` binades per row (some rows
    also get exact zeros): the row sums of squares round in f64 once the
    span passes the exact-sum bound, so only mean_sq's own order matches"""
    rng = np.random.default_rng(seed)
    m = rng.uniform(1.0, 2.0, shape) * rng.choice([-1.0, 1.0], shape)
    e = rng.integers(-span // 2, span - span // 2 + 1, shape)
    x = m * np.exp2(e)
    x[..., ::17] = 0.0
    return O.to_f64(O.from_f64(x, dt), dt)


@pytest.mark.parametrize("dt", (BF16, F16))
@pytest.mark.parametrize("dim", (64, 128, 256))
def test_wide_magnitude_rows(prims, dt, dim):
    """rows around and beyond the span where any summation order is exact
    (the 16-bit kernel's fast sum), and far beyond it (its ordered fallback)"""
    for span in (6, 11, 12, 13, 14, 15, 16, 17, 24):
        T, qh, kh = 9, 4, 2
        q = wide_rows(700 + span, (T, qh, dim), dt, span)
        k = wide_rows(800 + span, (T, kh, dim), dt, span)
        dq, dk = to_dev(O.from_f64(q, dt), dt), to_dev(O.from_f64(k, dt), dt)
        rc, rs = O.rope_table(1e6, dim, T, dt)
        prims.qk_norm_rope(dq, dk, EPS, QK, to_dev(O.from_f64(rc, dt), dt), to_dev(O.from_f64(rs, dt), dt))
        eq, ek = oracle_seq(q, k, dt, 1e6, dim, T, np.arange(T), True)
        assert same_bits(from_dev(dq, dt), O.from_f64(eq, dt)), span
        assert same_bits(from_dev(dk, dt), O.from_f64(ek, dt)), span


def test_errors(prims):
    import torch
    q = torch.zeros((2, 4, 128), dtype=torch.bfloat16, device="cuda:0")
    k = torch.zeros((2, 1, 128), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(Exception, match="head_dim"):
        prims.qk_norm_rope(q[:, :, :127].contiguous(), k[:, :, :127].contiguous(), EPS, QK)
    with pytest.raises(Exception, match="heads contiguous"):  # refused by the binding
        prims.qk_norm_rope(q[:, :, :127], k[:, :, :127], EPS, QK)
    with pytest.raises(Exception, match="v_cache"):
        prims.qk_norm_rope(q, k, EPS, QK, v_cache=k)
