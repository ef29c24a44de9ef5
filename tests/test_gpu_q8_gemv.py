"""GPU parity: the Q8_0 quantizer and the Q8_0 GEMV either side of dequant.

Quantizer: up_w (src/gpu/gpu_engine.cpp:2722-2755), bitwise against the oracle
restatement (oracle/oracle.cpp or_quantize_q8_0). Its agreement with llama.cpp's
quantize_row_q8_0, which is not vendored, is unpinned; the oracle is checked
against the rule's own invariants and its half-away-from-zero ties
(tests/test_oracle_math.py), and the device against the same exact ties here.
GEMV: k_gemv_q8 (src/gpu/gpu_engine.cpp:815-889) in f32 accumulation, so the
gate is a bound, not bits: |y - y64| <= 1e-5 * sum_i |w_i x_i| against the f64
sum of the same terms (each output adds at most ~90 f32 partial sums in
sequence: 80 per lane plus the 6-level lane tree).
"""
import numpy as np
import pytest

import oracle as O
from util import BF16, F32, from_dev, same_bits, to_dev

pytestmark = pytest.mark.gpu


def bf16_weights(seed, rows, n_in):
    w = O.normal(seed, (rows, n_in), 0.0, 0.05, BF16)
    wf = O.to_f64(w, BF16)
    wf[0, :32] = 0.0                       # an all-zero block: d = 0, q = 0
    wf[1, :32] = 1e-7 * np.arange(1, 33)   # subnormal f16 scale
    wf[2, :32] = np.arange(-16, 16) * 0.5  # half-integer weights (products are not ties: id = 127/8)
    wf[3, 32:64] = -wf[3, 32:64]
    return O.from_f64(wf, BF16)


@pytest.mark.parametrize("rows,n_in", ((64, 4096), (300, 160), (4, 32), (5, 96)))
def test_quantize_bitwise(prims, rows, n_in):
    """whole and partial 64-block waves (a wave quantizes 64 consecutive blocks)"""
    import torch
    w = bf16_weights(51, rows, n_in)
    rq, rd = O.quantize_q8_0(w)
    dq = torch.empty((rows, n_in), dtype=torch.int8, device="cuda:0")
    dd = torch.empty((rows, n_in // 32), dtype=torch.int16, device="cuda:0")
    prims.quantize_q8_0(to_dev(w, BF16), dq, dd)
    assert np.array_equal(dq.cpu().numpy(), rq)
    assert np.array_equal(dd.cpu().numpy().view(np.uint16), rd)


def test_quantize_exact_ties(prims):
    """blocks whose products x * id land exactly on k + 1/2 (id a power of two):
    lround's half away from zero, sign(x) (k + 1), not half-to-even"""
    import torch
    ks = np.array([0, 1, 2, 3, 4, 5, 62, 125, 0, 1, 2, 7, 9, 100, 126, 64,
                   0, 3, 6, 11, 20, 40, 80, 99, 1, 2, 4, 8, 16, 32, 120], np.int64)
    sign = np.where(np.arange(ks.size) % 3 == 1, -1, 1)
    rows = []
    for amax, idv in ((127.0, 1.0), (63.5, 2.0), (254.0, 0.5)):
        x = np.concatenate([[amax], sign * (ks + 0.5) / idv]).astype(np.float32)
        rows.append((x.view(np.uint32) >> 16).astype(np.uint16))
    w = np.tile(np.concatenate(rows), (4, 1))  # [4, 96]: three tie blocks per row
    dq = torch.empty((4, 96), dtype=torch.int8, device="cuda:0")
    dd = torch.empty((4, 3), dtype=torch.int16, device="cuda:0")
    prims.quantize_q8_0(to_dev(w, BF16), dq, dd)
    want = np.tile(np.concatenate([[127], sign * (ks + 1)]), 3)
    got = dq.cpu().numpy().astype(np.int64)
    for r in range(4):
        assert np.array_equal(got[r], want), r
    assert np.array_equal(dd.cpu().numpy().view(np.float16).astype(np.float64), np.tile([1.0, 0.5, 2.0], (4, 1)))


def gemv_case(prims, rows, n_in, B, blockdot, seed=52):
    import torch
    qs = O.int8_uniform(seed, (rows, n_in))
    d = O.from_f64(O.uniform(seed + 1, (rows, n_in // 32), 1e-3, 2e-2), O.F16)
    xs = O.normal(seed + 2, (B, n_in), 0.0, 1.0, BF16)
    x = O.to_f64(xs, BF16)
    dq, dd = torch.from_numpy(qs).to("cuda:0"), torch.from_numpy(d.view(np.int16)).to("cuda:0")
    dy = torch.zeros((B, rows), dtype=torch.float32, device="cuda:0")
    prims.gemv_q8_0(dq, dd, to_dev(xs, BF16), dy, blockdot)
    y = dy.cpu().numpy().astype(np.float64)
    scale = np.repeat(O.to_f64(d, O.F16), 32, axis=1)
    if blockdot:
        terms = qs.astype(np.float64) * scale       # d * q, summed per block first
    else:
        terms = O.dequant_q8_0(qs, d, BF16)          # bf16(q * d) per weight
    ref = x @ terms.T
    bound = np.abs(x) @ np.abs(terms).T
    err = np.abs(y - ref)
    assert np.all(err <= 1e-5 * bound + 1e-30), float((err / bound).max())


@pytest.mark.parametrize("B", (1, 3, 5))
@pytest.mark.parametrize("blockdot", (False, True))
def test_gemv(prims, B, blockdot):
    gemv_case(prims, 1000, 5120, B, blockdot)


@pytest.mark.parametrize("n_in", (32, 96, 160, 4160, 16384, 16448))
@pytest.mark.parametrize("blockdot", (False, True))
def test_gemv_widths(prims, n_in, blockdot):
    """input widths around the scale preload: rows whose scales are not whole
    32-bit words (96, 160), a last step with a few lanes (4160), the largest
    preloaded width (16384) and the next one (16448)"""
    gemv_case(prims, 37, n_in, 1, blockdot, seed=61)


def test_gemv_config5_shape(prims):
    """config 5's weight [25600, 5120] at decode (one token)"""
    gemv_case(prims, 25600, 5120, 1, False)


def test_quantize_dequant_gemv_chain(prims):
    """bf16 weight -> quantize -> GEMV equals GEMV over the oracle's quantization"""
    import torch
    rows, n_in = 512, 2048
    w = bf16_weights(53, rows, n_in)
    dq = torch.empty((rows, n_in), dtype=torch.int8, device="cuda:0")
    dd = torch.empty((rows, n_in // 32), dtype=torch.int16, device="cuda:0")
    prims.quantize_q8_0(to_dev(w, BF16), dq, dd)
    xs = O.normal(54, (2, n_in), 0.0, 1.0, BF16)
    dy = torch.zeros((2, rows), dtype=torch.float32, device="cuda:0")
    prims.gemv_q8_0(dq, dd, to_dev(xs, BF16), dy)
    rq, rd = O.quantize_q8_0(w)
    terms = O.dequant_q8_0(rq, rd, BF16)
    x = O.to_f64(xs, BF16)
    err = np.abs(dy.cpu().numpy() - x @ terms.T)
    assert np.all(err <= 1e-5 * (np.abs(x) @ np.abs(terms).T) + 1e-30)


def test_errors(prims):
    import torch
    q = torch.zeros((4, 48), dtype=torch.int8, device="cuda:0")
    d = torch.zeros((4, 1), dtype=torch.int16, device="cuda:0")
    x = torch.zeros((1, 48), dtype=torch.bfloat16, device="cuda:0")
    y = torch.zeros((1, 4), dtype=torch.float32, device="cuda:0")
    with pytest.raises(Exception, match="multiple of 32"):
        prims.gemv_q8_0(q, d, x, y)
