"""Helpers for moving oracle-format arrays to and from the GPU.

bf16/f16 storage is carried as uint16 bit patterns on the host (the oracle's
format) and as torch.bfloat16 / torch.float16 tensors on the device; the bits
are the same.
"""
import numpy as np

import oracle as O

F64, BF16, F16, F32 = O.F64, O.BF16, O.F16, O.F32


def torch_dtype(dt):
    import torch
    return {F64: torch.float64, BF16: torch.bfloat16, F16: torch.float16, F32: torch.float32}[dt]


def to_dev(arr, dt):
    import torch
    a = np.ascontiguousarray(arr)
    if dt in (BF16, F16):
        t = torch.from_numpy(a.view(np.int16)).view(torch_dtype(dt))
    else:
        t = torch.from_numpy(a.astype({F64: np.float64, F32: np.float32}[dt], copy=False))
    return t.to("cuda:0")


def from_dev(t, dt):
    import torch
    t = t.detach().to("cpu").contiguous()
    if dt in (BF16, F16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def bits16(x_f64, dt):
    """f64 values (already storage-valued) -> uint16 storage bits."""
    return O.from_f64(x_f64, dt)


def ulp_diff16(a_bits, b_bits):
    """|ordered(a) - ordered(b)| for bf16/f16 bit patterns (py/diff_lp.py:25-32 idea)."""
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    oa = np.where(a & 0x8000, 0x8000 - (a & 0x7fff), 0x8000 + a)
    ob = np.where(b & 0x8000, 0x8000 - (b & 0x7fff), 0x8000 + b)
    return np.abs(oa - ob)


def same_bits(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.dtype == np.float64:
        return np.array_equal(a.view(np.uint64), b.view(np.uint64))
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


def storage(seed, shape, dt, mean=0.0, std=1.0):
    """Seeded normal data at storage dtype, returned as (storage array, f64 values)."""
    s = O.normal(seed, shape, mean, std, dt)
    return s, O.to_f64(s, dt)


def is_nan16(bits, dt):
    b = bits.astype(np.uint32)
    if dt == BF16:
        return ((b & 0x7f80) == 0x7f80) & ((b & 0x7f) != 0)
    return ((b & 0x7c00) == 0x7c00) & ((b & 0x3ff) != 0)


def same_bits_or_nan(a, b, dt):
    """Bitwise equal, except that NaN only has to meet NaN: IEEE leaves the sign
    of a NaN produced by arithmetic unspecified, and x86 and gfx950 differ there."""
    if dt in (BF16, F16):
        na, nb = is_nan16(a, dt), is_nan16(b, dt)
    else:
        na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return same_bits(np.where(na, 0, a).astype(a.dtype), np.where(nb, 0, b).astype(b.dtype))
