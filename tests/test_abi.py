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
    assert lib.spc_subm_conv_preln(None, 0, None, 0, None, None, 1e-6, 1, None, None, 2, 0, 0, None, 0, 0, None, 4,
                                   64, 64, None, None) == -1
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


def test_header_is_plain_c_and_links(tmp_path):
    """include/spconv_amd.h compiles as C99 and a C program that calls host-only entry points links against the
    library and runs without a GPU (the header is what a cgo / JNI / N-API binding would include)."""
    src = tmp_path / "abi.c"
    src.write_text(r'''
#include <stdio.h>
#include "spconv_amd.h"
int main(void) {
  int b1, bk, s;
  if (spc_conv_cfg(1000, 64, 64, &b1, &bk, &s) != 0) return 1;
  if (spc_conv_cfg_autotune("/nonexistent.json", "NVIDIA H200", 1000, 64, 64, &b1, &bk, &s) == 0) return 2;
  if (spc_last_error() == 0 || spc_last_error()[0] == 0) return 3;
  if (spc_subm_conv(0, 0, 0, SPC_BF16, SPC_F32, 10, 64, 64, 0, 0) == 0) return 4;  /* null cache: an error */
  printf("%d %d %d\n", b1, bk, s);
  return 0;
}
''')
    exe = tmp_path / "abi"
    libdir = os.path.dirname(spconv_amd.LIB_PATH)
    cmd = (f"gcc -std=c99 -Wall -Werror -I{ROOT}/include {src} -o {exe} -L{libdir} -lspconv_amd "
           f"-Wl,-rpath,{libdir}")
    assert os.system(cmd) == 0, cmd
    out = os.popen(str(exe)).read()
    assert out.strip() == "128 64 1"


def test_diagnostics_without_gpu():
    """The timing and allocation diagnostics need no device: no conv call -> no kernel times; null pointers are
    errors; the allocation counters are readable."""
    lib = spconv_amd.load_library()
    assert lib.spc_kernel_timing(1) == 0
    n = ctypes.c_int(-1)
    assert lib.spc_kernel_times(None, 0, ctypes.byref(n)) == 0 and n.value == 0
    assert lib.spc_kernel_timing(0) == 0
    assert lib.spc_kernel_times(None, 0, None) == -1
    req, drv = spconv_amd.alloc_counts()
    assert req >= drv >= 0
    assert lib.spc_alloc_counts(None, None) == -1
