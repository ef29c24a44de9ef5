"""CPU checks of the C ABI library (no GPU needed): it loads, exports every
symbol include/mg_prims.h declares, and reports errors through mg_last_error
instead of crashing when no device is present."""
import ctypes
import os

import pytest

import mgprims


def test_library_exports_every_header_symbol():
    lib = mgprims.load_library()
    syms = mgprims.header_symbols()
    assert len(syms) >= 18
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_header():
    """every declared entry point has a ctypes signature in the binding"""
    assert set(mgprims.header_symbols()) == set(mgprims._SIGS)


def _header_params():
    """name -> parameter type strings, parsed from include/mg_prims.h"""
    import re
    with open(mgprims.HEADER) as f:
        text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(mg_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = params
    return out


def test_binding_matches_header_signatures():
    """each ctypes signature has the header's parameter count, and pointers, 64-bit
    integers, doubles and ints where the header has them (the ABI cannot drift)"""
    P, I64, D, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_int
    params = _header_params()
    assert set(params) == set(mgprims._SIGS)
    for name, (args, _) in mgprims._SIGS.items():
        hp = params[name]
        assert len(args) == len(hp), (name, len(args), len(hp))
        for a, h in zip(args, hp):
            if "*" in h:
                assert a in (P, ctypes.c_char_p) or issubclass(a, ctypes._Pointer), (name, h, a)
            elif h.startswith("int64_t"):
                assert a is I64, (name, h, a)
            elif h.startswith("double"):
                assert a is D, (name, h, a)
            elif h.startswith("int "):
                assert a is I, (name, h, a)


def test_open_reports_error_without_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = mgprims.load_library()
    h = ctypes.c_void_p()
    rc = lib.mg_open(0, None, 0, ctypes.byref(h))
    assert rc == -1
    assert lib.mg_last_error()  # a message, not a crash
    assert lib.mg_sync(None) == -1
    assert b"NULL context" in lib.mg_last_error()


def test_gfx950_code_object():
    """the library carries a gfx950 code object (built for MI355X only)"""
    with open(mgprims.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"gfx950" in blob
