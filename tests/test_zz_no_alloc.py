"""GPU check of spc_subdivide_noalloc, the allocation-free variant of spc_subdivide: called through the C ABI twice
in a row (the second call with fewer parents, so stale scratch contents from the first would show), each against
spc_subdivide's output on the same input and against the CPU oracle."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import spconv_amd as sp
from spconv_amd import workloads as W

pytestmark = pytest.mark.gpu


def _noalloc(lib, par, lg):
    n = par.shape[0]
    cc = torch.full((max(8 * n, 1), 4), -7, dtype=torch.int32, device=par.device)
    src = torch.full((max(8 * n, 1),), -7, dtype=torch.int32, device=par.device)
    m = torch.full((1,), -1, dtype=torch.int64, device=par.device)
    rc = lib.spc_subdivide_noalloc(ctypes.c_void_p(par.data_ptr()), ctypes.c_void_p(lg.data_ptr()), n,
                                   ctypes.c_void_p(cc.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                                   ctypes.c_void_p(m.data_ptr()))
    assert rc == 0, lib.spc_last_error()
    k = int(m.item())
    return cc[:k], src[:k]


def test_subdivide_noalloc_matches(gpu):
    lib = sp.load_library()
    sp.set_stream(torch.cuda.current_stream())
    cases = []
    for name, frac, seed in (("c5", 0.35, 21), ("c1", 0.6, 22)):  # second call smaller than the first
        par = W.shell_coords(W.CONFIGS[name])
        lg = W.keep_logits(len(par), frac, seed)
        lg[0, :] = np.array([-0.0, np.nan, np.inf, 6e-8, -6e-8, 0.0, -np.inf, 1.0], np.float16)
        cases.append((name, par, lg))
    for name, par, lg in cases:
        print(f"subdivide_noalloc case {name} n={len(par)}", flush=True)
        tp = torch.from_numpy(par).to(gpu)
        tl = torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16)
        torch.cuda.synchronize()
        before = sp.alloc_counts()
        nc, ns = _noalloc(lib, tp, tl)
        assert sp.alloc_counts() == before, "spc_subdivide_noalloc requested device memory from the library"
        rc, rs = sp.subdivide(tp, tl)
        assert nc.shape == rc.shape and ns.shape == rs.shape
        assert torch.equal(nc, rc) and torch.equal(ns, rs)
        oc, osrc = oracle.subdivide(par, lg)
        np.testing.assert_array_equal(nc.cpu().numpy(), oc)
        np.testing.assert_array_equal(ns.cpu().numpy(), osrc)


def test_subdivide_noalloc_empty_and_limit(gpu):
    lib = sp.load_library()
    sp.set_stream(torch.cuda.current_stream())
    m = torch.full((1,), -1, dtype=torch.int64, device=gpu)
    assert lib.spc_subdivide_noalloc(None, None, 0, None, None, ctypes.c_void_p(m.data_ptr())) == 0
    assert int(m.item()) == 0
    # one parent over the documented maximum fails before touching any pointer
    assert lib.spc_subdivide_noalloc(None, None, 4194305, None, None, ctypes.c_void_p(m.data_ptr())) == -1
    assert b"at most 4194304" in lib.spc_last_error()
