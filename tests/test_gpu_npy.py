"""GPU: .npy files to and from device tensors (mg_npy_load / mg_npy_save /
mg_npy_save_i64, the product path of oracle::Tensor's I/O, src/tensor.cpp:13-224).

  * every file under tests/golden/npy/ (the reference's own save_npy output and
    numpy's '<f8', '<f4', '<i8', '<i4', '|u1' files) loads to the f64 values the
    oracle's reader gives (pinned to the reference's load_npy in
    tests/test_oracle_npy.py), bitwise, and to bf16 / f16 / f32 as the twin's
    rounding of those values;
  * saving the loaded reference tensors writes the reference's bytes exactly,
    header padding included, for '<f8' tensors and the '<i8' vector;
  * a primitive runs on a loaded fixture: the weight-less RMSNorm of the
    reference-written [2, 3] tensor equals the oracle's on the same file, bit
    for bit (rows of d <= 128 sum in mean_sq's order).
"""
import os

import numpy as np
import pytest

import oracle as O
from util import BF16, F16, F32, F64, from_dev, same_bits

pytestmark = pytest.mark.gpu

NPY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "npy")
FILES = sorted(f for f in os.listdir(NPY) if f.endswith(".npy"))


@pytest.mark.parametrize("name", FILES)
def test_load_matches_the_reference_reader(prims, name):
    import torch
    path = os.path.join(NPY, name)
    want, _ = O.load_npy(path)
    got = prims.load_npy(path)
    assert got.dtype == torch.float64 and tuple(got.shape) == want.shape
    assert same_bits(got.cpu().numpy(), want)
    for tdt, dt in ((torch.float32, F32), (torch.bfloat16, BF16), (torch.float16, F16)):
        g = prims.load_npy(path, tdt)
        assert same_bits(from_dev(g, dt), O.from_f64(O.rnd(want, dt), dt)), (name, dt)


@pytest.mark.parametrize("name", [f for f in FILES if f.startswith("ref_")])
def test_save_writes_the_reference_bytes(prims, name, tmp_path):
    path = os.path.join(NPY, name)
    t = prims.load_npy(path)
    out = str(tmp_path / name)
    if name.startswith("ref_i64"):
        import torch
        prims.save_npy_i64(out, t.to(torch.int64))
    else:
        prims.save_npy(out, t)
    with open(path, "rb") as a, open(out, "rb") as b:
        assert a.read() == b.read()


def test_save_16bit_widens_exactly(prims, tmp_path):
    import torch
    x = torch.tensor([[1.5, -0.0078125, 65504.0], [float("inf"), -2.0 ** -24, 3.0]], dtype=torch.float16).cuda()
    p = str(tmp_path / "h.npy")
    prims.save_npy(p, x)
    r = np.load(p, allow_pickle=False)
    assert r.dtype == np.float64 and np.array_equal(r, x.cpu().double().numpy())


def test_primitive_on_a_loaded_fixture(prims):
    import torch
    x = prims.load_npy(os.path.join(NPY, "ref_f64_2x3.npy"))
    y = torch.empty_like(x)
    prims.rmsnorm_rows(O.WEIGHTLESS, x, None, 1e-6, y)
    xr, _ = O.load_npy(os.path.join(NPY, "ref_f64_2x3.npy"))
    want = O.rmsnorm_rows(O.WEIGHTLESS, xr, None, 1e-6, F64)
    assert same_bits(y.cpu().numpy(), want)


def test_load_checks_the_element_count(prims):
    import torch
    t = torch.empty(5, dtype=torch.float64, device="cuda:0")
    import ctypes
    rc = prims.lib.mg_npy_load(prims.h, os.fsencode(os.path.join(NPY, "ref_f64_7.npy")),
                               ctypes.c_void_p(t.data_ptr()), 5, 0)
    assert rc == -1 and b"7 values" in prims.lib.mg_last_error()
