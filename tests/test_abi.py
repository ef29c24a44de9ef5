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
