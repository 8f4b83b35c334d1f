"""Pins the CPU oracle (oracle/spc_oracle.c) with checks that do not restate its formulas:
hand-derived known answers, brute-force dictionary lookups, invariants, Python's stable sort, numpy reductions,
and torch.nn.functional.conv3d on the dense grid the sparse set is scattered into."""
import numpy as np
import pytest
import torch

import oracle
from spconv_amd import workloads as W

EMPTY = 0xFFFFFFFF


def offsets():
    return [(v // 9 - 1, v // 3 % 3 - 1, v % 3 - 1) for v in range(27)]


def small_shell(r=5.0, h=0.8, grid=16, seed=0, batches=1):
    """A few hundred voxels: a sphere shell per batch, Morton-sorted within each batch."""
    out = []
    for b in range(batches):
        cfg = W.Config("t", grid, 1, (r + b, r + b), False, h, 8, 8, "f32", "bias", seed + b, centred=True)
        c = W.shell_coords(cfg)
        c[:, 0] = b
        out.append(c)
    return np.concatenate(out, 0)


# ------------------------------------------------------------------------------------------ kernel map
def test_known_answer_four_voxels():
    # A=(1,1,1) B=(1,1,2) C=(2,1,1) D=(5,5,5); v = (dx+1)*9 + (dy+1)*3 + (dz+1)
    c = np.array([[0, 1, 1, 1], [0, 1, 1, 2], [0, 2, 1, 1], [0, 5, 5, 5]], np.int32)
    nbr, gray, binv, srt = oracle.build_neighbors(c, 8, 8, 8)
    exp = np.full((4, 27), EMPTY, np.uint32)
    exp[0, [13, 14, 22]] = [0, 1, 2]
    exp[1, [12, 13, 21]] = [0, 1, 2]
    exp[2, [4, 5, 13]] = [0, 1, 2]
    exp[3, 13] = 3
    np.testing.assert_array_equal(nbr, exp)
    np.testing.assert_array_equal(gray, [(1 << 13) | (1 << 14) | (1 << 22), (1 << 12) | (1 << 13) | (1 << 21),
                                         (1 << 4) | (1 << 5) | (1 << 13), 1 << 13])
    # decode of a mask = xor of the all-ones prefixes below each set bit (worked by hand)
    np.testing.assert_array_equal(binv, [2**23 - 1 - 2**14, 2**22 - 1 - 2**13, 2**14 - 1 - 2**5, 2**14 - 1])
    np.testing.assert_array_equal(srt, [2, 3, 1, 0])
    lst, seg = oracle.valid(gray, srt, 2)
    np.testing.assert_array_equal(lst, [4, 5, 13, 12, 13, 14, 21, 22])
    np.testing.assert_array_equal(seg, [0, 3, 8])


def brute_nbr(c, Wg, Hg, Dg):
    idx = {tuple(r): i for i, r in enumerate(c.tolist())}
    out = np.full((len(c), 27), EMPTY, np.uint32)
    for i, (b, x, y, z) in enumerate(c.tolist()):
        for v, (dx, dy, dz) in enumerate(offsets()):
            p = (b, x + dx, y + dy, z + dz)
            if 0 <= p[1] < Wg and 0 <= p[2] < Hg and 0 <= p[3] < Dg and p in idx:
                out[i, v] = idx[p]
    return out


@pytest.mark.parametrize("bounds", [(4096, 4096, 4096), (16, 16, 16), (12, 16, 9)])
def test_nbr_brute_force(bounds):
    c = small_shell(batches=2)
    keep = (c[:, 1] < bounds[0]) & (c[:, 2] < bounds[1]) & (c[:, 3] < bounds[2])
    c = c[keep]
    nbr, gray, binv, srt = oracle.build_neighbors(c, *bounds)
    np.testing.assert_array_equal(nbr, brute_nbr(c, *bounds))
    # mask = occupancy of the nbr row; centre always present
    mask = ((nbr != EMPTY) * (1 << np.arange(27, dtype=np.int64))).sum(1)
    np.testing.assert_array_equal(gray, mask)
    assert np.all(gray >> 13 & 1)


def test_nbr_symmetry_and_decode_and_sort():
    c = W.shell_coords(W.CONFIGS["c1"])
    nbr, gray, binv, srt = oracle.build_neighbors(c)
    n = len(c)
    i, v = np.nonzero(nbr != EMPTY)
    j = nbr[i, v].astype(np.int64)
    np.testing.assert_array_equal(nbr[j, 26 - v], i)  # nbr[i][v] = j  <=>  nbr[j][26-v] = i
    b = binv.astype(np.uint32)
    np.testing.assert_array_equal(b ^ (b >> 1), gray.astype(np.uint32))  # binary -> gray re-encodes the mask
    assert np.all(b < (1 << 27))
    np.testing.assert_array_equal(srt, sorted(range(n), key=lambda k: int(binv[k])))  # Python sort is stable


@pytest.mark.parametrize("B1", [1, 7, 32, 128, 100000])
def test_valid_lists(B1):
    c = W.shell_coords(W.CONFIGS["c1"])
    nbr, gray, binv, srt = oracle.build_neighbors(c)
    lst, seg = oracle.valid(gray, srt, B1)
    g = gray[srt].astype(np.int64)
    starts = np.arange(0, len(g), B1)
    ors = np.bitwise_or.reduceat(g, starts)
    bits = (ors[:, None] >> np.arange(27)) & 1
    np.testing.assert_array_equal(np.diff(seg), bits.sum(1))
    assert seg[0] == 0
    exp = np.nonzero(bits)[1]  # row-major nonzero: blocks in order, offsets ascending
    np.testing.assert_array_equal(lst, exp)


def test_empty_and_single():
    nbr, gray, binv, srt = oracle.build_neighbors(np.zeros((0, 4), np.int32))
    assert nbr.shape == (0, 27) and len(srt) == 0
    nbr, gray, binv, srt = oracle.build_neighbors(np.array([[0, 0, 0, 0]], np.int32))
    assert nbr[0, 13] == 0 and (nbr[0] != EMPTY).sum() == 1 and gray[0] == 1 << 13 and srt[0] == 0


# ------------------------------------------------------------------------------------------ conv
def dense_conv(c, x, w, b, grid):
    """Submanifold conv = zero-padded dense conv3d sampled at the active sites (one batch)."""
    ci, co = x.shape[1], w.shape[0]
    X = torch.zeros((1, ci, grid, grid, grid), dtype=torch.float64)
    X[0, :, c[:, 1], c[:, 2], c[:, 3]] = torch.from_numpy(x.astype(np.float64)).T
    Wt = torch.from_numpy(w.astype(np.float64)).reshape(co, 3, 3, 3, ci).permute(0, 4, 1, 2, 3).contiguous()
    Y = torch.nn.functional.conv3d(X, Wt, torch.from_numpy(b.astype(np.float64)), padding=1)
    return Y[0, :, c[:, 1], c[:, 2], c[:, 3]].T.numpy()


@pytest.mark.parametrize("act,res", [(0, False), (1, False), (0, True), (1, True)])
def test_conv_vs_dense_conv3d(act, res):
    cfg = W.CONFIGS["c1"]
    c = W.shell_coords(cfg)
    n = len(c)
    x = W.features(n, 32, 5)
    w, b = W.conv_params(cfg)
    r = W.features(n, 32, 6) if res else None
    nbr, _, _, _ = oracle.build_neighbors(c)
    y = oracle.conv(x, w, b, nbr, res=r, act=act)
    ref = dense_conv(c, x, w, b, cfg.grid)
    if act:
        ref = ref / (1.0 + np.exp(-ref))
    if res:
        ref = ref + r
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4)


def test_conv_row_subset_and_threads():
    cfg = W.CONFIGS["c1"]
    c = W.shell_coords(cfg)
    x = W.features(len(c), 32, 1)
    w, b = W.conv_params(cfg)
    nbr, _, _, _ = oracle.build_neighbors(c)
    full = oracle.conv(x, w, b, nbr, nthreads=1)
    rows = np.array([5, 0, len(c) - 1, 17])
    np.testing.assert_array_equal(oracle.conv(x, w, b, nbr, rows=rows, nthreads=3), full[rows])


def test_conv_centre_only_is_gemm():
    c = small_shell()
    x = W.features(len(c), 16, 2)
    rng = np.random.default_rng(3)
    w = np.zeros((24, 27, 16), np.float32)
    w[:, 13, :] = rng.standard_normal((24, 16))
    nbr, _, _, _ = oracle.build_neighbors(c)
    y = oracle.conv(x, w, None, nbr)
    np.testing.assert_allclose(y, x @ w[:, 13, :].T, rtol=1e-5, atol=1e-5)


def test_conv_isolated_voxels():
    c = np.array([[0, 0, 0, 0], [0, 10, 10, 10], [1, 0, 0, 0]], np.int32)
    x = W.features(3, 8, 4)
    w = np.random.default_rng(5).standard_normal((8, 27, 8)).astype(np.float32)
    nbr, _, _, _ = oracle.build_neighbors(c)
    np.testing.assert_allclose(oracle.conv(x, w, None, nbr), x @ w[:, 13, :].T, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------------------------------ subdivision
def test_subdivide():
    c = small_shell(batches=2)
    lg = W.keep_logits(len(c), 0.35, 9)
    lg[0, 0] = np.float16(-0.0)  # not > 0
    lg[0, 1] = np.float16(np.nan)  # not > 0
    lg[0, 2] = np.float16(np.inf)  # > 0
    lg[1, 3] = np.float16(6e-8)  # smallest subnormal, > 0
    oc, src = oracle.subdivide(c, lg)
    exp_c, exp_s = [], []
    for i in range(len(c)):
        for s in range(8):
            if float(lg[i, s]) > 0:
                b, x, y, z = c[i].tolist()
                exp_c.append([b, 2 * x + (s & 1), 2 * y + (s >> 1 & 1), 2 * z + (s >> 2 & 1)])
                exp_s.append(i * 8 + s)
    np.testing.assert_array_equal(oc, np.array(exp_c, np.int32).reshape(-1, 4))
    np.testing.assert_array_equal(src, exp_s)
    np.testing.assert_array_equal(oc[:, 1:] // 2, c[src // 8, 1:])


# ------------------------------------------------------------------------------------------ golden fixture
def load_golden():
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "small_shell.npz"))
    return {k: d[k] for k in d.files}


def bf16_bits_to_f32(a):
    return (a.astype(np.int32).astype(np.uint32) << 16).view(np.float32)


def test_oracle_matches_golden_fixture():
    """tests/golden/small_shell.npz was written by brute force and torch conv3d, not by the oracle."""
    g = load_golden()
    nbr, gray, binv, srt = oracle.build_neighbors(g["coords"])
    np.testing.assert_array_equal(nbr, g["nbr"])
    np.testing.assert_array_equal(gray, g["gray"])
    np.testing.assert_array_equal(binv, g["dec"])
    np.testing.assert_array_equal(srt, g["order"])
    for B1 in (32, 128):
        lst, seg = oracle.valid(gray, srt, B1)
        np.testing.assert_array_equal(lst, g[f"list{B1}"])
        np.testing.assert_array_equal(seg, g[f"seg{B1}"])
    x, w, b, r = (bf16_bits_to_f32(g[k]) for k in ("x", "w", "b", "r"))
    y = oracle.conv(x, w, b, nbr, res=r, act=1)
    np.testing.assert_allclose(y, g["y_silu_res"], rtol=1e-5, atol=1e-5)


def test_fdg_quads_known_answer():
    """Four voxels filling the 2x2 square x = 0, y, z in {0,1}: only voxel (0,0,0)'s x-axis edge has all four
    voxels ((0,0,0) (0,0,1) (0,1,1) (0,1,0), the x-axis edge offsets); a negative gate drops it."""
    c = np.array([[0, 0, 1, 1], [0, 0, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1]], np.int32)
    h = np.ones((4, 7), np.float32)
    quad, ok = oracle.fdg_quads(c, h, 8)
    assert ok.tolist() == [0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0]
    assert quad[3].tolist() == [1, 3, 0, 2]
    h[1, 3] = -0.0
    assert oracle.fdg_quads(c, h, 8)[1].sum() == 0
    # the same square one voxel below the grid's top: the quad needs (0,1,1), which R = 1 excludes
    assert oracle.fdg_quads(c, np.ones((4, 7), np.float32), 1)[1].sum() == 0


def test_lookup_oracle():
    c = np.array([[0, 1, 2, 3], [1, 1, 2, 3], [0, 4, 4, 4]], np.int32)
    q = np.array([[0, 1, 2, 3], [1, 1, 2, 3], [2, 1, 2, 3], [0, 4, 4, 4], [0, 4, 4, 5], [-1, 1, 2, 3],
                  [0, 8, 0, 0], [0, -1, 0, 0]], np.int32)
    assert oracle.lookup(c, q, 8, 8, 8).tolist() == [0, 1, -1, 2, -1, -1, -1, -1]
