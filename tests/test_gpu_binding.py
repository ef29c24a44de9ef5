"""GPU: row strides through the C ABI and the binding's checks.

Strided views (a row stride larger than the row, as a caller holding scores or
activations in a wider buffer passes them) give the same bits as the
contiguous call, on the vector path (stride a multiple of 8) and the
element-wise one. Views the ABI cannot express, and outputs too small for
the call, are refused by the binding before any pointer reaches a kernel.
"""
import math

import numpy as np
import pytest

import oracle as O
from util import BF16, F32, storage, to_dev

pytestmark = pytest.mark.gpu


def padded(t, pad):
    """a view of t's values inside a buffer whose rows are `pad` elements wider"""
    import torch
    big = torch.full(t.shape[:-1] + (t.shape[-1] + pad,), float("nan"), dtype=t.dtype, device=t.device)
    big[..., :t.shape[-1]] = t
    return big[..., :t.shape[-1]]


def bits(t):
    import torch
    return t.detach().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32).cpu().numpy()


@pytest.mark.parametrize("kc,pad", ((2048, 8), (2048, 3), (300, 16), (9000, 8), (9000, 5)))
@pytest.mark.parametrize("cap", (0.0, 30.0))
def test_softmax_row_strides(prims, kc, pad, cap):
    import torch
    heads, q = 3, 16
    xs, _ = storage(70, (heads, q, kc), F32, 0.0, 3.0)
    x = to_dev(xs, F32)
    y = torch.empty((heads, q, kc), dtype=torch.bfloat16, device="cuda:0")
    prims.softmax_rows(x, y, 1 / math.sqrt(128), O.MASK_CAUSAL, 0, kc - q, cap)
    xv = padded(x, pad)
    yv = padded(torch.zeros_like(y), pad + 1)
    prims.softmax_rows(xv, yv, 1 / math.sqrt(128), O.MASK_CAUSAL, 0, kc - q, cap)
    torch.cuda.synchronize()
    assert np.array_equal(bits(yv), bits(y))
    # the padding of the output rows (NaN from padded()) is left alone
    assert torch.all(torch.isnan(yv.as_strided((heads * q, pad + 1), (kc + pad + 1, 1), kc)))


@pytest.mark.parametrize("dim,pad", ((5120, 8), (5120, 1), (128, 64)))
def test_residual_rmsnorm_row_strides(prims, dim, pad):
    import torch
    import mgprims
    rows = 33
    h0 = to_dev(O.normal(71, (rows, dim), 0, 1, BF16), BF16)
    x = to_dev(O.normal(72, (rows, dim), 0, 1, BF16), BF16)
    w = to_dev(O.normal(73, (dim,), 1, 0.05, BF16), BF16)
    h, y = h0.clone(), torch.empty_like(h0)
    prims.residual_rmsnorm(mgprims.CENTERED, h, x, w, 1e-6, y)
    hv, xv, yv = padded(h0, pad), padded(x, pad + 2), padded(torch.empty_like(y), pad + 4)
    prims.residual_rmsnorm(mgprims.CENTERED, hv, xv, w, 1e-6, yv)
    torch.cuda.synchronize()
    assert np.array_equal(bits(hv), bits(h)) and np.array_equal(bits(yv), bits(y))


def test_binding_refuses_what_the_abi_cannot_take(prims):
    import torch
    import mgprims
    dev = "cuda:0"
    g = torch.zeros((64, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(mgprims.MgError, match="contiguous"):
        prims.swiglu(g.t(), g, torch.empty_like(g))
    with pytest.raises(mgprims.MgError, match="elements"):
        prims.swiglu(g, g, torch.empty((10,), dtype=torch.bfloat16, device=dev))
    with pytest.raises(mgprims.MgError, match="dtype"):
        prims.swiglu(g, g.float(), torch.empty_like(g))
    with pytest.raises(mgprims.MgError, match="cuda"):
        prims.swiglu(g, g.cpu(), torch.empty_like(g))
    with pytest.raises(mgprims.MgError, match="stride 1"):
        prims.rmsnorm_rows(mgprims.WEIGHTLESS, g.t(), None, 1e-6, torch.empty((128, 64), dtype=g.dtype, device=dev))
    s = torch.zeros((2, 16, 64), dtype=torch.float32, device=dev)
    with pytest.raises(mgprims.MgError, match="row stride"):
        prims.softmax_rows(s.transpose(0, 1), torch.empty((16, 2, 64), dtype=torch.bfloat16, device=dev), 1.0)
    with pytest.raises(mgprims.MgError, match="shape"):
        prims.softmax_rows(s, torch.empty((2, 16, 32), dtype=torch.bfloat16, device=dev), 1.0)
    qs = torch.zeros((4, 64), dtype=torch.int8, device=dev)
    with pytest.raises(mgprims.MgError, match="scales"):
        prims.dequant_q8_0(qs, torch.zeros((4, 1), dtype=torch.float16, device=dev), torch.empty((4, 64), dtype=g.dtype,
                                                                                                  device=dev))
