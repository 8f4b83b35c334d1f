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


# FlexiDualGrid edge offsets per axis (reference c_edge_off, src/mesh.cu:20-24): the 4 voxels around voxel i's
# edge along axis a, as (dx, dy, dz) added to (x, y, z).
FDG_EDGE = (((0, 0, 0), (0, 0, 1), (0, 1, 1), (0, 1, 0)),
            ((0, 0, 0), (1, 0, 0), (1, 0, 1), (0, 0, 1)),
            ((0, 0, 0), (0, 1, 0), (1, 1, 0), (1, 0, 0)))


def lookup(coords: np.ndarray, query: np.ndarray, W: int, H: int, D: int) -> np.ndarray:
    """Row of each (b,x,y,z) query in coords, -1 if absent or outside [0,W)x[0,H)x[0,D) (a Python dict as the hash;
    the probe of src/mesh.cu:14-19 with the batch kept in the key)."""
    rows = {tuple(int(v) for v in c): i for i, c in enumerate(np.asarray(coords))}
    out = np.full(len(query), -1, np.int32)
    for j, (b, x, y, z) in enumerate(np.asarray(query).tolist()):
        if b >= 0 and 0 <= x < W and 0 <= y < H and 0 <= z < D:
            out[j] = rows.get((b, x, y, z), -1)
    return out


def fdg_quads(coords: np.ndarray, h: np.ndarray, R: int):
    """(quad int32 [3n,4], ok int32 [3n]) of k_fdg_quads (src/mesh.cu:36-45) for one batch: e = 3i + a is kept when
    h[i,3+a] > 0 and the 4 voxels at FDG_EDGE[a] exist inside [0,R)^3; quad rows of dropped edges are -1 here (the
    reference leaves them unwritten). Pure Python: small cases only."""
    c = np.asarray(coords)
    rows = {(int(x), int(y), int(z)): i for i, (_, x, y, z) in enumerate(c.tolist())}
    n = len(c)
    quad = np.full((3 * n, 4), -1, np.int32)
    ok = np.zeros(3 * n, np.int32)
    for i in range(n):
        _, x, y, z = (int(v) for v in c[i])
        for a in range(3):
            if not h[i, 3 + a] > 0:
                continue
            r = []
            for dx, dy, dz in FDG_EDGE[a]:
                p = (x + dx, y + dy, z + dz)
                r.append(rows.get(p, -1) if all(0 <= v < R for v in p) else -1)
            if min(r) >= 0:
                ok[3 * i + a] = 1
                quad[3 * i + a] = r
    return quad, ok
