"""CPU: the library's .npy header reader (mg_npy_info, the product path of
src/tensor.cpp's load_npy) on files the reference's own save_npy /
save_npy_i64 wrote (tests/golden/npy/ref_*.npy) and on numpy's files of every
element type load_npy reads: the stored descr and shape. No GPU is needed;
what the loader makes of the data is tests/test_gpu_npy.py."""
import os

import numpy as np
import pytest

import mgprims

NPY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "npy")
FILES = sorted(f for f in os.listdir(NPY) if f.endswith(".npy"))


@pytest.mark.parametrize("name", FILES)
def test_header_matches_numpy(name):
    path = os.path.join(NPY, name)
    descr, shape = mgprims.npy_info(path)
    a = np.load(path, allow_pickle=False)
    assert shape == a.shape
    assert descr == a.dtype.str


def test_missing_and_foreign_files_fail(tmp_path):
    with pytest.raises(mgprims.MgError, match="cannot open"):
        mgprims.npy_info(str(tmp_path / "absent.npy"))
    p = tmp_path / "text.npy"
    p.write_bytes(b"not an array")
    with pytest.raises(mgprims.MgError, match="not an .npy file"):
        mgprims.npy_info(str(p))
    q = tmp_path / "fortran.npy"
    np.save(q, np.asfortranarray(np.ones((3, 2))))
    with pytest.raises(mgprims.MgError, match="Fortran"):
        mgprims.npy_info(str(q))
