"""The C-ABI library loads and exports every symbol include/zeromoe.h declares
(no compute calls: runs without a GPU)."""
import ctypes
import os
import re

from zeromoe_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    txt = open(os.path.join(ROOT, "include", "zeromoe.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b((?:zm|launch)_[A-Za-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_header_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    syms = header_symbols()
    assert len(syms) >= 14
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(header_symbols()) == set(_lib.SIGNATURES)


def test_host_only_calls():
    L = _lib.lib()
    assert L.zm_mul_mat_id_negative_skip() == 1
    assert L.zm_mul_mat_id_negative_skip_batched() == 1
    assert b"gfx950" in L.zm_version()
    import numpy as np
    import zm_oracle as O

    g = np.zeros(256, np.uint64)
    L.zm_iq2xxs_builtin_grid(g.ctypes.data)
    np.testing.assert_array_equal(g, O.iq2xxs_grid())  # library stand-in == oracle stand-in
