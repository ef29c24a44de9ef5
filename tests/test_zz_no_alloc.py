"""GPU: mg_vocab_reduce_noalloc, the vocab pass that allocates nothing (its
partials in the library's fixed device scratch array instead of a context's
workspace), against mg_vocab_reduce on the same logits: lse bitwise, argmax
and top-K ids and values identical. Two calls in a row, the second smaller,
so stale partials of the first would show; then a call whose partials do not
fit the array must fail before launching, and a call after it still works.
Everything goes through the C ABI (ctypes), with no context for the new entry
point."""
import ctypes

import numpy as np
import pytest

import oracle as O
from util import BF16, F32, to_dev

pytestmark = pytest.mark.gpu


def noalloc(lib, stream, logits, K):
    import torch
    rows, V = logits.shape
    dev = logits.device
    lse = torch.full((rows,), np.nan, dtype=torch.float64, device=dev)
    am = torch.full((rows,), -7, dtype=torch.int64, device=dev)
    ti = torch.full((rows, K), -7, dtype=torch.int64, device=dev)
    tv = torch.full((rows, K), np.nan, dtype=torch.float32, device=dev)
    code = {torch.float32: 3, torch.bfloat16: 1}[logits.dtype]
    rc = lib.mg_vocab_reduce_noalloc(ctypes.c_void_p(stream), ctypes.c_void_p(logits.data_ptr()), 0, rows, V, code, K,
                                     ctypes.c_void_p(lse.data_ptr()), ctypes.c_void_p(am.data_ptr()),
                                     ctypes.c_void_p(ti.data_ptr()), ctypes.c_void_p(tv.data_ptr()))
    return rc, lse, am, ti, tv


def same(a, b):
    return np.array_equal(a.cpu().numpy().view(np.uint8), b.cpu().numpy().view(np.uint8))


@pytest.mark.parametrize("dt", (F32, BF16))
def test_noalloc_matches_context_entry_point(prims, dt):
    import torch
    lib = prims.lib
    stream = torch.cuda.current_stream().cuda_stream
    for rows, V, K, seed in ((64, 201088, 64, 61), (5, 50001, 40, 62)):  # the second call is smaller
        L = O.normal(seed, (rows, V), 0.0, 4.0, dt)
        if rows > 8:
            Lf = O.to_f64(L, dt)
            Lf[3, 1000:1010] = Lf[3].max() + 1.0  # ties at the top: lower index first
            Lf[7, :] = -np.inf
            L = O.from_f64(Lf, dt)
        dL = to_dev(L, dt)
        print(f"noalloc vs context: dt={dt} rows={rows} V={V} K={K}", flush=True)
        rc, lse, am, ti, tv = noalloc(lib, stream, dL, K)
        assert rc == 0, lib.mg_last_error().decode()
        rlse, ram, rti, rtv = prims.vocab_reduce(dL, K)
        torch.cuda.synchronize()
        assert same(lse, rlse) and same(am, ram) and same(ti, rti) and same(tv, rtv)


def test_noalloc_rejects_partials_beyond_the_scratch(prims):
    import torch
    lib = prims.lib
    stream = torch.cuda.current_stream().cuda_stream
    # 1024 rows x 50 chunks need 1024 * 50 * 2216 bytes (113 MB) > 16 MiB: refused, nothing launched
    big = torch.zeros((1024, 201088), dtype=torch.float32, device="cuda:0")
    rc, *_ = noalloc(lib, stream, big, 64)
    assert rc == -1 and b"fixed scratch array" in lib.mg_last_error()
    del big
    # a call that fits still works afterwards
    L = O.normal(63, (3, 4096), 0.0, 4.0, F32)
    dL = to_dev(L, F32)
    rc, lse, am, ti, tv = noalloc(lib, stream, dL, 8)
    assert rc == 0
    rlse, ram, rti, rtv = prims.vocab_reduce(dL, 8)
    torch.cuda.synchronize()
    assert same(lse, rlse) and same(am, ram) and same(ti, rti) and same(tv, rtv)


def test_noalloc_on_a_side_stream_keeps_the_current_device(prims):
    """the call runs on its stream's device (here the one GPU, through a stream other
    than torch's current one) and leaves the thread's current device as it was"""
    import torch
    lib = prims.lib
    L = O.normal(63, (4, 30000), 0.0, 4.0, F32)
    dL = to_dev(L, F32)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    before = torch.cuda.current_device()
    with torch.cuda.stream(side):
        rc, lse, am, ti, tv = noalloc(lib, side.cuda_stream, dL, 16)
    assert rc == 0, lib.mg_last_error().decode()
    side.synchronize()
    assert torch.cuda.current_device() == before
    rlse, ram, rti, rtv = prims.vocab_reduce(dL, 16)
    torch.cuda.synchronize()
    assert same(lse, rlse) and same(am, ram) and same(ti, rti) and same(tv, rtv)
