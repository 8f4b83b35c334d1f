"""ctypes bindings of the CPU oracle (spc_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only as the checker
or the CPU baseline. The product library (trellis2-cuda_amd) never calls it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
_lib = None

EMPTY = 0xFFFFFFFF


def build() -> None:
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(_LIB)
        P = ctypes.c_void_p
        L.orc_build_neighbors.argtypes = [P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P]
        L.orc_build_neighbors.restype = ctypes.c_int
        L.orc_valid.argtypes = [P, P, ctypes.c_int64, ctypes.c_int, P, P]
        L.orc_valid.restype = ctypes.c_int64
        L.orc_conv.argtypes = [P, P, P, P, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P,
                               ctypes.c_int]
        L.orc_conv.restype = ctypes.c_int
        L.orc_subdivide.argtypes = [P, P, ctypes.c_int64, P, P]
        L.orc_subdivide.restype = ctypes.c_int64
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def build_neighbors(coords: np.ndarray, W: int = 4096, H: int = 4096, D: int = 4096):
    """Returns (nbr u32 [n,27], gray i32 [n], bin i32 [n], sorted i32 [n])."""
    c = np.ascontiguousarray(coords, dtype=np.int32)
    n = len(c)
    nbr = np.empty((n, 27), np.uint32)
    gray = np.empty(n, np.int32)
    binv = np.empty(n, np.int32)
    srt = np.empty(n, np.int32)
    rc = lib().orc_build_neighbors(_p(c), n, W, H, D, _p(nbr), _p(gray), _p(binv), _p(srt))
    assert rc == 0
    return nbr, gray, binv, srt


def valid(gray: np.ndarray, sorted_: np.ndarray, B1: int):
    """Returns (list[:L] i32, seg i32 [nb+1])."""
    n = len(gray)
    nb = (n + B1 - 1) // B1
    lst = np.empty(max(27 * nb, 1), np.int32)
    seg = np.empty(nb + 1, np.int32)
    g = np.ascontiguousarray(gray, np.int32)
    s = np.ascontiguousarray(sorted_, np.int32)
    L = lib().orc_valid(_p(g), _p(s), n, B1, _p(lst), _p(seg))
    return lst[:L].copy(), seg


def conv(x, w, b, nbr, res=None, act: int = 0, rows=None, nthreads: int | None = None) -> np.ndarray:
    """fp32 gather-accumulate: y = act(sum_v x[nbr[:,v]] w[:,v,:]^T + b) [+ res]; returns [len(rows) or n, Co]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    b = None if b is None else np.ascontiguousarray(b, np.float32)
    res = None if res is None else np.ascontiguousarray(res, np.float32)
    nbr = np.ascontiguousarray(nbr, np.uint32)
    co, _, ci = w.shape
    if rows is not None:
        rows = np.ascontiguousarray(rows, np.int64)
        nrows = len(rows)
    else:
        nrows = len(nbr)
    out = np.empty((nrows, co), np.float32)
    nt = nthreads or os.cpu_count() or 1
    rc = lib().orc_conv(_p(x), _p(w), _p(b), _p(res), act, _p(nbr), _p(rows), nrows, ci, co, _p(out), nt)
    assert rc == 0
    return out


def subdivide(coords: np.ndarray, logits_f16: np.ndarray):
    """Returns (child coords i32 [m,4], src i32 [m])."""
    c = np.ascontiguousarray(coords, np.int32)
    lg = np.ascontiguousarray(logits_f16, np.float16).view(np.uint16)
    m = lib().orc_subdivide(_p(c), _p(lg), len(c), None, None)
    oc = np.empty((m, 4), np.int32)
    src = np.empty(m, np.int32)
    lib().orc_subdivide(_p(c), _p(lg), len(c), _p(oc), _p(src))
    return oc, src
