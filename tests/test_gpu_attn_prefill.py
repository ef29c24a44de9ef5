"""GPU envelope: tiled prefill attention over the KV ring.

Reference: the GPU engine's --flash-prefill tier (attention_flash,
src/gpu/gpu_engine.cpp:3292-3372; k_flash_softmax 1481-1545; k_flash_finish
1547-1560). Like that tier this is a tile-wise summation schedule with bf16
probabilities in the p.v product, gated on an envelope, not bits. The oracle is
exact f64 attention over the same bf16 q, K, V (scaling taken as the f32 value
the kernel uses). Each weight enters the p.v product as bf16(e), within 2^-8
of e relative (bf16 carries 8 significant bits; round to nearest), while the
normalizer sums e itself, so per output
|o - o64| <= (2^-8 + 2e-5) * sum_j p_j |v_j|; the 2e-5 covers the f32 scores,
exp2 and the per-tile rescales.
"""
import math

import numpy as np
import pytest

import oracle as O
from util import BF16, to_dev

pytestmark = pytest.mark.gpu
TOL = 2.0 ** -8 + 2e-5


def prefill_case(prims, T, nq, nkv, D, slots, pos0, window=0, seed=101, scaling=None, heads=None, rows=None):
    """keys 0..pos0+T-1 live in the ring (key j in slot j % slots); check the
    given heads and query rows (all by default) against f64 attention"""
    q = O.normal(seed, (T, nq, D), 0.0, 1.0, BF16)
    kc = O.normal(seed + 1, (slots, nkv, D), 0.0, 1.0, BF16)
    vc = O.normal(seed + 2, (slots, nkv, D), 0.0, 1.0, BF16)
    scaling = 1.0 / math.sqrt(D) if scaling is None else scaling
    out = prims.attn_prefill(to_dev(q, BF16), to_dev(kc, BF16), to_dev(vc, BF16), pos0, scaling, window)
    out = out.cpu().numpy().astype(np.float64)
    qf, K, Vv = O.to_f64(q, BF16), O.to_f64(kc, BF16), O.to_f64(vc, BF16)
    s32 = float(np.float32(scaling))
    hpg = nq // nkv
    heads = range(nq) if heads is None else heads
    rows = range(T) if rows is None else rows
    worst = 0.0
    for h in heads:
        g = h // hpg
        for t in rows:
            p_ = pos0 + t
            lo = max(0, p_ - window + 1) if window > 0 else 0
            sl = np.arange(lo, p_ + 1) % slots
            Kg, Vg = K[sl, g, :], Vv[sl, g, :]
            s = (Kg @ qf[t, h]) * s32
            p = np.exp(s - s.max())
            p /= p.sum()
            ref = p @ Vg
            bound = p @ np.abs(Vg)
            err = np.abs(out[t, h] - ref)
            assert np.all(err <= TOL * bound), (h, t, float((err / bound).max()))
            worst = max(worst, float((err / bound).max()))
    return worst


@pytest.mark.parametrize("nq,nkv,D", ((40, 8, 128), (8, 8, 64), (16, 2, 128), (7, 7, 64)))
def test_shapes(prims, nq, nkv, D):
    prefill_case(prims, 100, nq, nkv, D, 128, 0)


@pytest.mark.parametrize("hpg", (1, 2, 3, 4, 5, 6, 8))
@pytest.mark.parametrize("D", (64, 128))
def test_group_sizes(prims, hpg, D):
    """every query-head count per KV head (one wave per head of the group)"""
    prefill_case(prims, 70, 2 * hpg, 2, D, 80, 0, seed=110 + hpg)


@pytest.mark.parametrize("hpg", (9, 10, 16))
def test_large_groups(prims, hpg):
    """groups past 8 heads over several work-groups (9 -> 3 x 3, 10 -> 2 x 5, 16 -> 2 x 8)"""
    prefill_case(prims, 70, 2 * hpg, 2, 128, 80, 0, seed=160 + hpg)


def test_real_model_heads(prims):
    """32 query / 2 kv heads, head_dim 128, a chunk after a 200-token prefix"""
    prefill_case(prims, 130, 32, 2, 128, 400, 200, seed=170)


def test_chunked_prefill(prims):
    """a second chunk: rows at positions 50..126 see the first chunk's keys too"""
    prefill_case(prims, 77, 40, 8, 128, 160, 50, seed=120)


def test_window_and_ring(prims):
    """sliding window of 64 keys over a 128-slot ring that has wrapped"""
    prefill_case(prims, 60, 40, 8, 128, 128, 200, window=64, seed=121)
    prefill_case(prims, 96, 16, 2, 64, 200, 0, window=33, seed=122)


def test_window_ring_many_steps(prims):
    """a 256-key window over a 600-slot ring, positions 1000..1299: nine 64-key
    steps per tile, the ring wrapping (slot 0 again at key 1200) inside the
    chunk, so steps staged two ahead straddle the wrap"""
    prefill_case(prims, 300, 8, 2, 128, 600, 1000, window=256, seed=123)
    prefill_case(prims, 300, 10, 2, 64, 600, 1000, window=200, seed=124)


def test_short_and_ragged(prims):
    """one row, rows that end inside a 16-row tile, a 32-row tile boundary"""
    for T in (1, 15, 17, 31, 32, 33):
        prefill_case(prims, T, 8, 2, 128, 64, 0, seed=130 + T)


def test_peaked_scores(prims):
    """scaling 1: the running maxima move late and the lazy rescale runs"""
    prefill_case(prims, 300, 8, 2, 128, 512, 0, scaling=1.0, seed=140)


@pytest.mark.parametrize("scaling", (0.35, 0.6))
def test_reference_kept_below_threshold(prims, scaling):
    """a row's reference maximum moves only when a new maximum passes it by more
    than 8 in log2 units; at these scalings the maxima of later steps often pass
    the first one by a few units without moving it, so weights between 1 and 2^8
    reach the sums and the p.v product"""
    prefill_case(prims, 257, 8, 2, 128, 512, 0, scaling=scaling, seed=141)


@pytest.mark.parametrize("scaling", (-1.0 / math.sqrt(128), -1.0, 0.0, 1e-30))
def test_scaling_signs(prims, scaling):
    """the kernel multiplies by |scaling| inside the exponent: a negative
    scaling (q enters negated, so the weights favour the least similar keys),
    zero (every attended key weighs the same) and a tiny one"""
    prefill_case(prims, 90, 8, 2, 128, 128, 20, scaling=scaling, seed=145)


def test_config3_prefill_sampled(prims):
    """config 3's prompt: 4096 tokens, 40 q / 8 kv heads, causal; a sample of
    heads and rows against f64 (the full f64 check is minutes of numpy)"""
    rows = list(range(0, 40)) + list(range(2040, 2056)) + list(range(4060, 4096))
    prefill_case(prims, 4096, 40, 8, 128, 4096, 0, seed=150, heads=(0, 4, 5, 23, 39), rows=rows)


def test_errors(prims):
    import torch
    q = torch.zeros((4, 6, 128), dtype=torch.bfloat16, device="cuda:0")
    kc = torch.zeros((16, 4, 128), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(Exception, match="multiple"):
        prims.attn_prefill(q, kc, kc, 0, 0.1)
    q = torch.zeros((20, 8, 128), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(Exception, match="cache ring"):
        prims.attn_prefill(q, kc, kc, 0, 0.1)
