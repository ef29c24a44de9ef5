"""GPU parity: RoPE table and rotate-half application.

Reference: build_rope_table (src/muse_glimmer.hpp:625-674) and apply_rope
(681-705) over (token, head) as 809-819. Both are bitwise against the oracle
(whose table and rotation are themselves bitwise against the reference's
compiled code, tests/test_oracle_ref.py).
"""
import numpy as np
import pytest

import oracle as O
from util import BF16, F16, F32, F64, from_dev, same_bits, storage, to_dev, torch_dtype

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
@pytest.mark.parametrize("theta,dim,T", ((1e6, 128, 4096), (5e5, 128, 2048), (1e4, 64, 300)))
def test_table_bitwise(prims, dt, theta, dim, T):
    co, si = prims.build_rope_table(theta, dim, T, torch_dtype(dt))
    rc, rs = O.rope_table(theta, dim, T, dt)
    assert same_bits(from_dev(co, dt), O.from_f64(rc, dt))
    assert same_bits(from_dev(si, dt), O.from_f64(rs, dt))


def rope_case(prims, dt, T, qh, kh, dim, theta=1e6, positions=None, pos0=0, table_T=None, specials=False):
    table_T = table_T or T
    rc, rs = O.rope_table(theta, dim, table_T, dt)
    dco, dsi = to_dev(O.from_f64(rc, dt), dt), to_dev(O.from_f64(rs, dt), dt)
    qs, q = storage(6, (T, qh, dim), dt)
    ks, k = storage(7, (T, kh, dim), dt)
    if specials:
        big = 3e38 if dt == BF16 else 6e4
        q[0, 0, 3] = np.nan                 # NaN in the low half: both rotated outputs NaN
        q[0, 1, 70] = np.inf                # inf in the high half
        q[1, 2, 5], q[1, 2, 69] = big, big  # products and sums near overflow
        q[2, 3, :] = -0.0                   # signed zeros
        k[3, 0, 10] = -np.inf
        qs, q = O.from_f64(q, dt), O.to_f64(O.from_f64(q, dt), dt)
        ks, k = O.from_f64(k, dt), O.to_f64(O.from_f64(k, dt), dt)
    dq, dk = to_dev(qs, dt), to_dev(ks, dt)
    dpos = None
    if positions is not None:
        import torch
        dpos = torch.from_numpy(np.asarray(positions, np.int64)).to("cuda:0")
        pos = np.asarray(positions, np.int64)
    else:
        pos = np.arange(pos0, pos0 + T, dtype=np.int64)
    prims.apply_rope(dq, dk, dco, dsi, dpos, pos0)
    rq = O.apply_rope(q, rc, rs, pos, dt)
    rk = O.apply_rope(k, rc, rs, pos, dt)
    return from_dev(dq, dt), from_dev(dk, dt), rq, rk


@pytest.mark.parametrize("dt", (BF16, F16, F32, F64))
def test_apply_bitwise(prims, dt):
    q, k, rq, rk = rope_case(prims, dt, 257, 40, 8, 128)
    assert same_bits(q, O.from_f64(rq, dt))
    assert same_bits(k, O.from_f64(rk, dt))


def test_special_values_bf16(prims):
    """NaN, inf, overflow and signed zeros: bitwise (bf16's NaN is the one pattern 0x7FC0)"""
    q, k, rq, rk = rope_case(prims, BF16, 9, 8, 2, 128, specials=True)
    assert same_bits(q, O.from_f64(rq, BF16))
    assert same_bits(k, O.from_f64(rk, BF16))


def test_config3_full(prims):
    """Config 3 RoPE: q [4096, 40, 128], k [4096, 8, 128] bf16, theta 1e6, positions 0..4095."""
    q, k, rq, rk = rope_case(prims, BF16, 4096, 40, 8, 128)
    assert same_bits(q, O.from_f64(rq, BF16))
    assert same_bits(k, O.from_f64(rk, BF16))


def test_positions_array_and_offset(prims):
    pos = [5, 0, 4095, 17, 17, 1000, 2, 3]
    q, k, rq, rk = rope_case(prims, BF16, len(pos), 32, 2, 128, 5e5, positions=pos, table_T=4096)
    assert same_bits(q, O.from_f64(rq, BF16)) and same_bits(k, O.from_f64(rk, BF16))
    q, k, rq, rk = rope_case(prims, BF16, 16, 32, 2, 128, 5e5, pos0=100, table_T=4096)
    assert same_bits(q, O.from_f64(rq, BF16)) and same_bits(k, O.from_f64(rk, BF16))


def test_odd_head_dim_scalar_path(prims):
    q, k, rq, rk = rope_case(prims, BF16, 33, 3, 1, 18)  # half = 9: not a multiple of 8
    assert same_bits(q, O.from_f64(rq, BF16)) and same_bits(k, O.from_f64(rk, BF16))


def test_q_only(prims):
    rc, rs = O.rope_table(1e6, 128, 64, BF16)
    qs, q = storage(8, (64, 4, 128), BF16)
    dq = to_dev(qs, BF16)
    prims.apply_rope(dq, None, to_dev(O.from_f64(rc, BF16), BF16), to_dev(O.from_f64(rs, BF16), BF16))
    rq = O.apply_rope(q, rc, rs, np.arange(64), BF16)
    assert same_bits(from_dev(dq, BF16), O.from_f64(rq, BF16))


def test_errors(prims):
    import mgprims
    import torch
    q = torch.zeros((8, 2, 128), dtype=torch.bfloat16, device="cuda:0")
    co = torch.zeros((4, 64), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(mgprims.MgError, match="outside the table"):
        prims.apply_rope(q, None, co, co, None, 0)
    with pytest.raises(mgprims.MgError, match="theta"):
        prims.build_rope_table(-1.0, 128, 16, torch.bfloat16)
