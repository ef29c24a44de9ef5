"""CPU: the oracle's .npy I/O (the reference's fixture format, src/tensor.h:11-48,
src/tensor.cpp:13-224) against files the reference's own save_npy / save_npy_i64
wrote (tests/golden/npy/ref_*.npy, via oracle/_ref) and against numpy.

Pins: the committed reference files load back exactly; writing the same tensor
gives the same bytes (so the header text and its padding to 64 bytes match);
numpy reads what the oracle writes; every element type the reference reads
('<f8', '<f4', '<i8', '<i4', '|u1', written by numpy) widens to the same f64
values the reference's load_npy gives (tests/golden/npy.npz).
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NPY = os.path.join(GOLD, "npy")


def ref_file(name):
    return os.path.join(NPY, name)


def test_round_trip(tmp_path):
    """tests/test_npy.cpp:8-30: a [2, 3] f64 tensor and an i64 vector round-trip"""
    p = str(tmp_path / "oracle_test.npy")
    t = (0.1 * np.arange(6.0) - 0.25).reshape(2, 3)
    O.save_npy(p, t)
    r, descr = O.load_npy(p)
    assert descr == "<f8" and r.shape == (2, 3)
    assert np.array_equal(r, t)
    O.save_npy(p, np.array([5, -1, 262143], np.int64))
    ri, descr = O.load_npy(p)
    assert descr == "<i8" and ri.shape == (3,) and ri[2] == 262143.0 and ri[1] == -1.0


@pytest.mark.parametrize("name,shape", (("ref_f64_2x3.npy", (2, 3)), ("ref_f64_2x1x5.npy", (2, 1, 5)),
                                        ("ref_f64_7.npy", (7,))))
def test_reference_files_load_and_rewrite_bytewise(tmp_path, name, shape):
    got, descr = O.load_npy(ref_file(name))
    assert descr == "<f8" and got.shape == shape
    want = np.load(ref_file(name), allow_pickle=False)  # numpy as the independent reader
    assert np.array_equal(got.view(np.uint64), want.astype(np.float64).view(np.uint64))
    if name == "ref_f64_2x3.npy":
        assert np.array_equal(got, (0.1 * np.arange(6.0) - 0.25).reshape(2, 3))
    out = str(tmp_path / name)
    O.save_npy(out, got)
    with open(out, "rb") as a, open(ref_file(name), "rb") as b:
        assert a.read() == b.read()


def test_reference_i64_file(tmp_path):
    got, descr = O.load_npy(ref_file("ref_i64_3.npy"))
    assert descr == "<i8" and np.array_equal(got, [5.0, -1.0, 262143.0])
    out = str(tmp_path / "i.npy")
    O.save_npy(out, np.array([5, -1, 262143], np.int64))
    with open(out, "rb") as a, open(ref_file("ref_i64_3.npy"), "rb") as b:
        assert a.read() == b.read()


def test_headers_pad_to_64_and_numpy_reads_them(tmp_path):
    rng = np.random.default_rng(3)
    for shape in ((), (1,), (17,), (3, 5), (2, 3, 4, 5), (1, 1, 1, 1, 1, 1, 1, 1)):
        a = rng.normal(0, 1, shape)
        p = str(tmp_path / "a.npy")
        O.save_npy(p, a)
        with open(p, "rb") as f:
            raw = f.read()
        hl = raw[8] | (raw[9] << 8)
        assert raw[:8] == b"\x93NUMPY\x01\x00" and (10 + hl) % 64 == 0 and raw[10 + hl - 1:10 + hl] == b"\n"
        assert np.array_equal(np.load(p, allow_pickle=False), a)
        b, _ = O.load_npy(p)
        assert b.shape == a.shape and np.array_equal(b, a)


def test_numpy_written_types_widen_as_the_reference_reads_them():
    ref = np.load(os.path.join(GOLD, "npy.npz"))
    for name, descr in (("np_f4", "<f4"), ("np_i4", "<i4"), ("np_i8", "<i8"), ("np_u1", "|u1"), ("np_f8", "<f8")):
        got, d = O.load_npy(ref_file(name + ".npy"))
        assert d == descr
        assert np.array_equal(got, ref[name]), name
        assert np.array_equal(got, np.load(ref_file(name + ".npy"), allow_pickle=False).astype(np.float64)), name


def test_rejects_what_the_reference_rejects(tmp_path):
    p = str(tmp_path / "f.npy")
    np.save(p, np.asfortranarray(np.ones((3, 2))), allow_pickle=False)
    with pytest.raises(O.NpyError, match="fortran"):
        O.load_npy(p)
    np.save(p, np.ones(4, np.float16), allow_pickle=False)
    with pytest.raises(O.NpyError, match="unsupported descr <f2"):
        O.load_npy(p)
    with open(p, "wb") as f:
        f.write(b"not a numpy file")
    with pytest.raises(O.NpyError, match="not an npy"):
        O.load_npy(p)
    with pytest.raises(O.NpyError, match="cannot open"):
        O.load_npy(str(tmp_path / "missing.npy"))


@pytest.mark.skipif(not O.Ref.available(), reason="oracle/_ref not built (needs /root/reference)")
def test_reference_reads_oracle_files(tmp_path):
    R = O.Ref()
    a = np.random.default_rng(4).normal(0, 1e5, (4, 3, 2))
    p = str(tmp_path / "a.npy")
    O.save_npy(p, a)
    assert np.array_equal(R.load_npy(p, a.shape), a)


@pytest.mark.skipif(not O.Ref.available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("shape", ((), (1,), (12,), (3, 4), (2, 1, 3, 1), tuple([2] * 8), (1000, 3)))
def test_same_bytes_as_the_reference_writer(tmp_path, shape):
    R = O.Ref()
    a = np.random.default_rng(len(shape)).normal(0, 1, shape)
    pa, pb = str(tmp_path / "a.npy"), str(tmp_path / "b.npy")
    O.save_npy(pa, a)
    R.save_npy(pb, a)
    with open(pa, "rb") as f, open(pb, "rb") as g:
        assert f.read() == g.read()
    v = np.arange(-3, int(np.prod(shape)) - 3, dtype=np.int64)
    O.save_npy(pa, v)
    R.save_npy(pb, v)
    with open(pa, "rb") as f, open(pb, "rb") as g:
        assert f.read() == g.read()
