"""CPU: the C-ABI library loads and exports every symbol include/mpq_amd.h declares."""
import ctypes
import os
import re

import pytest

from mpq_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = set()
    for fname in os.listdir(os.path.join(ROOT, "include")):
        if fname.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fname)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(mpq_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared_symbols()
    assert "mpq_e8p12_map" in names
    assert set(names) == set(_lib.exported_symbols()), "Python binding table out of sync with the header"


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmpq_amd.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_symbols():
        assert hasattr(lib, name), name


def test_invalid_argument_reported_without_gpu():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmpq_amd.so not built")
    lib = _lib.load()
    # negative n is rejected on the host before any HIP call
    rc = lib.mpq_e8p12_map(None, -1, None, 1, None, None, 0.0, None, None, None, None, None, None)
    assert rc == -1
    assert b"n must be" in lib.mpq_last_error()
    lib.mpq_clear_error()
    assert lib.mpq_last_error() == b""


def test_pointer_arguments_stay_alive_until_the_call_returns():
    """_lib.ptr(x.contiguous()) must not free the temporary before the library reads it: a later
    argument's temporary could otherwise take the same block."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmpq_amd.so not built")
    import gc
    import weakref

    import torch

    t = torch.empty(4)
    ref = weakref.ref(t)
    _lib.ptr(t)
    del t
    gc.collect()
    assert ref() is not None
    _lib.call("mpq_last_error_code")
    gc.collect()
    assert ref() is None
