"""CPU-side checks of the boundary: the built library loads without a GPU and exports every entry point that
include/spconv_amd.h declares; no compute call is made here."""
import ctypes
import os
import re

import pytest

import spconv_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    txt = open(os.path.join(ROOT, "include", "spconv_amd.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(spc_[a-z_0-9]+)\s*\(", txt)))


def test_header_lists_binding_symbols():
    assert declared() == sorted(spconv_amd.SYMBOLS)


def test_library_exports_declared_symbols():
    lib = spconv_amd.load_library()
    for name in declared():
        assert hasattr(lib, name), name
    nm = os.popen(f"nm -D --defined-only {spconv_amd.LIB_PATH}").read()
    exported = set(re.findall(r" T (spc_\w+)", nm))
    assert exported == set(declared())


def test_error_convention_without_gpu():
    lib = spconv_amd.load_library()
    # argument checks fire before any device work: -1 and a message, never an exception across the ABI
    assert lib.spc_build_neighbors(None, 10, 8, 8, 8, None) == -1
    assert b"null" in lib.spc_last_error()
    assert lib.spc_subm_conv(None, None, None, 2, 0, 4, 32, 64, None, None) == -1
    assert b"cache is null" in lib.spc_last_error()
    b1, bk, s = spconv_amd.spconv_cfg(400000, 256, 256)
    assert (b1, bk, s) == (128, 64, 1)
    assert spconv_amd.spconv_cfg(1000, 32, 64)[1] == 32


def test_no_oracle_in_product():
    """The product library and binding never reference the oracle."""
    pkg = os.path.join(ROOT, "trellis2-cuda_amd")
    for dp, _, fs in os.walk(pkg):
        for f in fs:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                src = open(os.path.join(dp, f)).read()
                assert "import oracle" not in src and "liboracle" not in src and "orc_" not in src, f
    assert "orc_" not in os.popen(f"nm -D {spconv_amd.LIB_PATH}").read()
