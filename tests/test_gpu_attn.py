"""GPU envelope: split-K decode attention over the KV ring.

Reference: the GPU engine's flash-decode split + combine
(src/gpu/gpu_engine.cpp:1690-1857) over the cache layout of k_kv_append
(481-492); like the reference's own split-K path this is gated on a numerical
envelope, not bits. The oracle is exact f64 attention over the same bf16 q, K,
V (scaling taken as the f32 value the kernel uses); the gate per output is
|o - o64| <= 5e-5 * sum_j p_j |v_j| (f32 dot products, online softmax and the
split merge stay well inside it).
"""
import math

import numpy as np
import pytest

import oracle as O
from util import BF16, to_dev

pytestmark = pytest.mark.gpu


def attn_case(prims, nq, nkv, D, slots, qpos, window=0, seed=61, scaling=None):
    q = O.normal(seed, (nq, D), 0.0, 1.0, BF16)
    kc = O.normal(seed + 1, (slots, nkv, D), 0.0, 1.0, BF16)
    vc = O.normal(seed + 2, (slots, nkv, D), 0.0, 1.0, BF16)
    scaling = 1.0 / math.sqrt(D) if scaling is None else scaling
    out = prims.attn_decode(to_dev(q, BF16), to_dev(kc, BF16), to_dev(vc, BF16), qpos, scaling, window)
    out = out.cpu().numpy().astype(np.float64)
    lo = max(0, qpos - window + 1) if window > 0 else 0
    pos = np.arange(lo, qpos + 1)
    sl = pos % slots
    qf, K, Vv = O.to_f64(q, BF16), O.to_f64(kc, BF16), O.to_f64(vc, BF16)
    s32 = float(np.float32(scaling))
    hpg = nq // nkv
    for h in range(nq):
        g = h // hpg
        Kg, Vg = K[sl, g, :], Vv[sl, g, :]
        s = (Kg @ qf[h]) * s32
        p = np.exp(s - s.max())
        p /= p.sum()
        ref = p @ Vg
        bound = p @ np.abs(Vg)
        err = np.abs(out[h] - ref)
        assert np.all(err <= 5e-5 * bound), (h, float((err / bound).max()))


@pytest.mark.parametrize("nq,nkv,D", ((40, 8, 128), (8, 8, 128), (16, 2, 64), (7, 7, 64)))
def test_shapes(prims, nq, nkv, D):
    attn_case(prims, nq, nkv, D, 5000, 4999)


@pytest.mark.parametrize("hpg", (1, 2, 3, 4, 6, 8))
@pytest.mark.parametrize("D", (64, 128))
def test_group_sizes(prims, hpg, D):
    """every query-head count per KV head the matrix-core tiles pad to 16"""
    attn_case(prims, 2 * hpg, 2, D, 3000, 2999, seed=80 + hpg)


@pytest.mark.parametrize("hpg", (9, 12, 16, 20, 32))
def test_large_groups(prims, hpg):
    """groups past 8 heads: up to 16 per wave (the MFMA's columns), larger
    groups over several waves of a divisor (20 -> 2 x 10, 32 -> 2 x 16)"""
    attn_case(prims, 2 * hpg, 2, 128, 3000, 2999, seed=90 + hpg)


def test_real_model_heads(prims):
    """32 query / 2 kv heads, head_dim 128 (the checkpoint's attention shape)"""
    attn_case(prims, 32, 2, 128, 8192, 8000, seed=95)
    attn_case(prims, 32, 2, 128, 1024, 5000, window=1024, seed=96)


def test_peaked_scores(prims):
    """scaling 1: scores spread over tens of units, so the running maxima move
    late in the splits and the lazy rescale runs"""
    attn_case(prims, 40, 8, 128, 8192, 8191, scaling=1.0, seed=91)


def test_long_unaligned(prims):
    """a context that is not a multiple of the step or split length (longer
    splits for long contexts), ending part-way through a step"""
    attn_case(prims, 40, 8, 128, 40960, 39999 - 7, seed=92)
    attn_case(prims, 40, 8, 128, 70000, 65536 + 17, window=60001, seed=93)


def test_window_and_ring(prims):
    """sliding window of 1000 keys; a ring of 3000 slots at position 7000"""
    attn_case(prims, 40, 8, 128, 5000, 4321, window=1000)
    attn_case(prims, 40, 8, 128, 3000, 7000, window=2000)


def test_short_contexts(prims):
    for qpos in (0, 1, 63, 64, 511, 512, 513):
        attn_case(prims, 40, 8, 128, 1024, qpos, seed=70 + qpos)


def test_decode_131072(prims):
    """config 4's decode context: one token against 131072 cached keys"""
    attn_case(prims, 40, 8, 128, 131072, 131071)


def test_errors(prims):
    import torch
    q = torch.zeros((6, 128), dtype=torch.bfloat16, device="cuda:0")
    kc = torch.zeros((16, 4, 128), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(Exception, match="multiple"):
        prims.attn_decode(q, kc, kc, 5, 0.1)
    q = torch.zeros((8, 128), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(Exception, match="cache ring"):
        prims.attn_decode(q, kc, kc, 100, 0.1)
