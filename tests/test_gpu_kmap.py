"""GPU parity of the hash table, 27-offset kernel map, gray-code sorted order, valid lists and subdivision:
bit-exact against the CPU oracle (and a hand-derived known answer) on the same coordinates."""
import numpy as np
import pytest
import torch

import oracle
import spconv_amd as sp
from spconv_amd import workloads as W

pytestmark = pytest.mark.gpu

_coords_cache = {}


def coords(name):
    if name not in _coords_cache:
        if name == "c5_children":
            cfg = W.CONFIGS["c5"]
            par = coords("c5")
            oc, _ = oracle.subdivide(par, W.keep_logits(len(par), cfg.keep_frac, cfg.seed))
            _coords_cache[name] = oc
        else:
            _coords_cache[name] = W.shell_coords(W.CONFIGS[name])
    return _coords_cache[name]


def gpu_map(c, dev, bounds=(4096, 4096, 4096)):
    t = torch.from_numpy(np.ascontiguousarray(c, np.int32)).to(dev)
    cache = sp.build_neighbors(t, *bounds)
    nbr, gray, srt = cache.tensors()
    return cache, nbr.cpu().numpy().view(np.uint32), gray.cpu().numpy(), srt.cpu().numpy()


def check_map(c, dev, bounds=(4096, 4096, 4096), B1s=(32, 128)):
    print(f"kmap case n={len(c)} bounds={bounds}", flush=True)
    cache, nbr, gray, srt = gpu_map(c, dev, bounds)
    onbr, ogray, _, osrt = oracle.build_neighbors(c, *bounds)
    np.testing.assert_array_equal(nbr, onbr)
    np.testing.assert_array_equal(gray, ogray)
    np.testing.assert_array_equal(srt, osrt)
    for B1 in B1s:
        lst, seg = cache.valid(B1)
        olst, oseg = oracle.valid(ogray, osrt, B1)
        np.testing.assert_array_equal(seg.cpu().numpy(), oseg)
        np.testing.assert_array_equal(lst.cpu().numpy(), olst)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5", "c5_children", "c4"])
def test_kmap_configs(gpu, name):
    check_map(coords(name), gpu, B1s=(32, 128, 1000))


def test_kmap_known_answer(gpu):
    c = np.array([[0, 1, 1, 1], [0, 1, 1, 2], [0, 2, 1, 1], [0, 5, 5, 5]], np.int32)
    cache, nbr, gray, srt = gpu_map(c, gpu, (8, 8, 8))
    exp = np.full((4, 27), 0xFFFFFFFF, np.uint32)
    exp[0, [13, 14, 22]] = [0, 1, 2]
    exp[1, [12, 13, 21]] = [0, 1, 2]
    exp[2, [4, 5, 13]] = [0, 1, 2]
    exp[3, 13] = 3
    np.testing.assert_array_equal(nbr, exp)
    np.testing.assert_array_equal(srt, [2, 3, 1, 0])
    lst, seg = cache.valid(2)
    np.testing.assert_array_equal(lst.cpu().numpy(), [4, 5, 13, 12, 13, 14, 21, 22])
    np.testing.assert_array_equal(seg.cpu().numpy(), [0, 3, 8])


def test_kmap_edges(gpu):
    # empty set
    cache, nbr, gray, srt = gpu_map(np.zeros((0, 4), np.int32), gpu)
    assert nbr.shape == (0, 27) and len(srt) == 0
    lst, seg = cache.valid(128)
    assert seg.cpu().tolist() == [0]
    # one voxel at the grid corner
    check_map(np.array([[0, 0, 0, 0]], np.int32), gpu, (4, 4, 4), B1s=(1, 128))
    # several batches, neighbours cut by tight bounds, voxels on every face of the box
    c = W.shell_coords(W.Config("e", 12, 1, (5, 5), False, 1.0, 8, 8, "f32", "bias", 3, centred=True))
    cs = []
    for b in range(3):
        cc = c.copy()
        cc[:, 0] = b
        cs.append(cc)
    c = np.concatenate(cs)
    check_map(c, gpu, (12, 12, 12), B1s=(1, 3, 64, 128))
    # a full dense block: every interior voxel has all 27 neighbours, ties everywhere in the sort
    g = np.stack(np.meshgrid(np.arange(9), np.arange(9), np.arange(9), indexing="ij"), -1).reshape(-1, 3)
    c = np.concatenate([np.zeros((len(g), 1), np.int32), g.astype(np.int32)], 1)
    check_map(c, gpu, (9, 9, 9))


def test_kmap_random_permutation(gpu):
    # row order is not Morton: the stable sort must still reproduce ties in row order
    c = coords("c2").copy()
    c = c[np.random.default_rng(0).permutation(len(c))]
    check_map(c, gpu)


@pytest.mark.parametrize("n", [524288, 524289])
def test_kmap_sort_paths(gpu, n):
    """The stable sort switches from the tile look-back form (at most 256 tiles of 2048 keys) to count/scan/scatter
    passes above it: both sides of the switch, on a permuted prefix of the c4 shell (ties in non-Morton order)."""
    c = coords("c4")[:n].copy()
    c = c[np.random.default_rng(1).permutation(n)]
    print(f"sort path n={n}", flush=True)
    check_map(c, gpu, B1s=(128,))


@pytest.mark.parametrize("limit", ["0", "1"])
def test_kmap_sort_unpublished_digit_sums(gpu, monkeypatch, limit):
    """The sort's digit-scan workgroups wait a bounded number of polls for the lower digits' published sums and
    then sum those digits' tile counts themselves. With the bound forced to 0 (every lower sum recomputed) or 1
    (a mix of both paths) the order must stay bit-exact: the wait bound may never change the result."""
    monkeypatch.setenv("SPCONV_SORT_SPIN_LIMIT", limit)
    c = coords("c4")[:600000].copy()
    c = c[np.random.default_rng(2).permutation(len(c))]
    print(f"sort spin limit {limit} n={len(c)}", flush=True)
    check_map(c, gpu, B1s=(128,))


@pytest.mark.parametrize("name", ["c1", "c5"])
def test_subdivide(gpu, name):
    par = coords(name)
    lg = W.keep_logits(len(par), 0.35, 11)
    lg[0, :] = np.array([-0.0, np.nan, np.inf, 6e-8, -6e-8, 0.0, -np.inf, 1.0], np.float16)
    oc, osrc = oracle.subdivide(par, lg)
    tc = torch.from_numpy(par).to(gpu)
    tl = torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16)
    gc, gs = sp.subdivide(tc, tl)
    np.testing.assert_array_equal(gc.cpu().numpy(), oc)
    np.testing.assert_array_equal(gs.cpu().numpy(), osrc)


def test_kmap_golden_fixture(gpu):
    """Against tests/golden/small_shell.npz (brute-force kernel map, shuffled rows, two batches)."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "small_shell.npz"))
    cache, nbr, gray, srt = gpu_map(g["coords"], gpu)
    np.testing.assert_array_equal(nbr, g["nbr"])
    np.testing.assert_array_equal(gray, g["gray"])
    np.testing.assert_array_equal(srt, g["order"])
    for B1 in (32, 128):
        lst, seg = cache.valid(B1)
        np.testing.assert_array_equal(lst.cpu().numpy(), g[f"list{B1}"])
        np.testing.assert_array_equal(seg.cpu().numpy(), g[f"seg{B1}"])


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_lookup(gpu, name):
    """Coordinate queries against the kept hash: every voxel finds its own row; shifted, other-batch, out-of-grid
    and negative queries match a dictionary lookup."""
    c = coords(name)
    print(f"lookup case {name} n={len(c)}", flush=True)
    R = 64 if name == "c2" else 32
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu), R, R, R, keep_hash=True)
    rng = np.random.default_rng(3)
    q = np.concatenate([c, c + np.array([0, 1, 0, 0], np.int32), c + np.array([1, 0, 0, 0], np.int32),
                        rng.integers(-2, R + 2, size=(5000, 4)).astype(np.int32) * np.array([0, 1, 1, 1], np.int32)])
    got = sp.lookup(cache, torch.from_numpy(q).to(gpu)).cpu().numpy()
    np.testing.assert_array_equal(got[:len(c)], np.arange(len(c)))
    np.testing.assert_array_equal(got, oracle.lookup(c, q, R, R, R))
    with pytest.raises(RuntimeError):  # no hash kept
        sp.lookup(sp.build_neighbors(torch.from_numpy(c).to(gpu), R, R, R), torch.from_numpy(q[:4]).to(gpu))
    empty = sp.build_neighbors(torch.zeros((0, 4), dtype=torch.int32, device=gpu), R, R, R, keep_hash=True)
    assert sp.lookup(empty, torch.from_numpy(q[:9]).to(gpu)).cpu().tolist() == [-1] * 9


@pytest.mark.parametrize("permute", [False, True])
def test_lookup_large(gpu, permute):
    """C4-size kept hash (a table of >= 2^22 slots, sized on the device from the brick-key runs of the input): every
    voxel finds its own row, and +x / +y shifted queries of a sample match a sorted-key search. Permuted input has
    about one run per voxel, so the table keeps its full size."""
    c = coords("c4")
    if permute:
        c = c[np.random.default_rng(5).permutation(len(c))]
    print(f"lookup_large permute={permute} n={len(c)}", flush=True)
    R = 1024
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu), R, R, R, keep_hash=True)
    got = sp.lookup(cache, torch.from_numpy(c).to(gpu)).cpu().numpy()
    np.testing.assert_array_equal(got, np.arange(len(c)))
    key = lambda a: ((a[:, 0].astype(np.int64) * R + a[:, 1]) * R + a[:, 2]) * R + a[:, 3]
    k = key(c)
    srt = np.argsort(k)
    ks = k[srt]
    samp = c[np.random.default_rng(6).choice(len(c), 200000, replace=False)]
    for d in ([0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, -1]):
        q = samp + np.array(d, np.int32)
        inside = ((q[:, 1:] >= 0) & (q[:, 1:] < R)).all(1)
        qk = key(np.where(inside[:, None], q, 0))
        pos = np.minimum(np.searchsorted(ks, qk), len(ks) - 1)
        want = np.where(inside & (ks[pos] == qk), srt[pos], -1)
        np.testing.assert_array_equal(sp.lookup(cache, torch.from_numpy(q).to(gpu)).cpu().numpy(), want)


@pytest.mark.parametrize("name,R", [("c1", 32), ("c1", 20)])
def test_fdg_quads(gpu, name, R):
    """Quads from the kernel map equal the reference rule evaluated with a dictionary hash (ok flags everywhere,
    quad rows where ok), including voxels cut by a tight grid bound."""
    c = coords(name)
    c = c[(c[:, 1:] < R).all(1)]
    print(f"fdg case {name} R={R} n={len(c)}", flush=True)
    h = np.random.default_rng(5).standard_normal((len(c), 7)).astype(np.float32)
    cache = sp.build_neighbors(torch.from_numpy(np.ascontiguousarray(c)).to(gpu), R, R, R)
    quad, ok = sp.fdg_quads(cache, torch.from_numpy(h).to(gpu))
    oq, ook = oracle.fdg_quads(c, h, R)
    ok = ok.cpu().numpy()
    np.testing.assert_array_equal(ok, ook)
    assert ok.sum() > 0
    np.testing.assert_array_equal(quad.cpu().numpy()[ok == 1], oq[ook == 1])


def dense_volume(c, attrs, X, Y, Z):
    """attrs of the sparse voxels scattered into a zero volume laid out for torch's 5-D grid_sample: [1, C, Z, Y, X]
    (grid's last dimension is (x, y, z) -> (W, H, D))."""
    vol = torch.zeros((1, attrs.shape[1], Z, Y, X), dtype=torch.float64)
    ci = torch.from_numpy(c.astype(np.int64))
    vol[0, :, ci[:, 3], ci[:, 2], ci[:, 1]] = attrs.double().T
    return vol


def torch_sample(vol, pts, X, Y, Z):
    """torch.nn.functional.grid_sample, trilinear, align_corners=False, zero padding: continuous voxel coordinate p
    (voxel i spans [i, i+1)) normalizes to 2p/size - 1."""
    size = torch.tensor([X, Y, Z], dtype=torch.float64)
    g = (2 * pts.double() / size - 1).view(1, 1, 1, -1, 3)
    return torch.nn.functional.grid_sample(vol, g, mode="bilinear", padding_mode="zeros", align_corners=False)[
        0, :, 0, 0, :].T


@pytest.mark.parametrize("name", ["c1", "dense"])
def test_grid_sample(gpu, name):
    """The bake's trilinear sample map + weighted sum on the kept hash, against torch's grid_sample on the dense
    volume the sparse attributes are scattered into (absent voxels read zero there, as EMPTY corners do here): points
    inside, on voxel centres and faces, and past the grid edge. Rows bit-exact against dictionary lookups of the 8
    corners; weights sum to 1 where all corners exist; the normalized form divides by the present weights' sum."""
    if name == "c1":
        c = coords("c1")
        X = Y = Z = 32
    else:
        g = np.stack(np.meshgrid(np.arange(6), np.arange(5), np.arange(7), indexing="ij"), -1).reshape(-1, 3)
        c = np.concatenate([np.zeros((len(g), 1), np.int64), g], 1).astype(np.int32)
        X, Y, Z = 6, 5, 7
    rng = np.random.default_rng(3)
    L = 4000
    pts = rng.uniform(-1.0, [X + 1, Y + 1, Z + 1], size=(L, 3)).astype(np.float32)
    pts[:200] = c[rng.integers(0, len(c), 200), 1:] + 0.5  # voxel centres: one corner with weight 1
    pts[200:300, 0] = np.floor(pts[200:300, 0]) + 0.5      # on a centre plane along x
    attrs = torch.from_numpy(rng.standard_normal((len(c), 6)).astype(np.float32))
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu), X, Y, Z, keep_hash=True)
    tp = torch.from_numpy(pts).to(gpu)
    nb, wt = sp.grid_sample_map(cache, tp)
    y = sp.grid_sample_sum(attrs.to(gpu), nb, wt).cpu()
    ref = torch_sample(dense_volume(c, attrs, X, Y, Z), torch.from_numpy(pts), X, Y, Z)
    assert torch.allclose(y.double(), ref, atol=2e-5, rtol=1e-5), float((y.double() - ref).abs().max())
    # rows: dictionary lookups of the corners of floor(p - 0.5)
    d = {tuple(r[1:]): i for i, r in enumerate(c)}
    base = np.floor(pts.astype(np.float64) - 0.5).astype(np.int64)
    exp = np.full((L, 8), -1, np.int64)
    for v in range(8):
        off = np.array([v >> 2, (v >> 1) & 1, v & 1])
        q = base + off
        exp[:, v] = [d.get(tuple(p), -1) for p in q]
    nbh, wth = nb.cpu().numpy(), wt.cpu().numpy()
    np.testing.assert_array_equal(nbh, exp)
    assert np.all(wth[exp < 0] == 0)
    full = (exp >= 0).all(1)
    assert np.allclose(wth[full].sum(1), 1.0, atol=1e-6)
    assert np.all(wth[:200].max(1) == 1.0)  # centres
    nb2, wt2 = sp.grid_sample_map(cache, tp, normalize=True)
    assert torch.equal(nb2, nb)
    s = wth.sum(1, keepdims=True)
    some = s[:, 0] > 0
    assert np.allclose(wt2.cpu().numpy()[some], wth[some] / s[some], rtol=1e-6, atol=1e-7)
    # another batch index finds nothing
    nb3, wt3 = sp.grid_sample_map(cache, tp, batch=1)
    assert bool((nb3 == -1).all()) and bool((wt3 == 0).all())


@pytest.mark.parametrize("name", ["c1", "c5"])
def test_subdivide_build(gpu, name):
    """subdivide_build (no host sync between the subdivision and the map build: launches sized for the 8n-child
    capacity, kernels stopped at the device-side count) equals subdivide followed by build_neighbors: children, src,
    nbr, gray, sorted and the valid lists bit for bit, the children's map against the oracle, and a conv on either
    cache gives identical outputs."""
    par = coords(name)
    cfg = W.CONFIGS["c5"]
    lg = W.keep_logits(len(par), cfg.keep_frac, cfg.seed)
    tc = torch.from_numpy(par).to(gpu)
    tl = torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16)
    print(f"subdivide_build case {name} parents={len(par)}", flush=True)
    cc, src, cache = sp.subdivide_build(tc, tl)
    rc, rs = sp.subdivide(tc, tl)
    assert torch.equal(cc, rc) and torch.equal(src, rs)
    ref = sp.build_neighbors(rc.contiguous())
    a, b = cache.tensors(), ref.tensors()
    for x, y in zip(a, b):
        assert x.shape == y.shape and torch.equal(x, y)
    for B1 in (32, 128):
        for x, y in zip(cache.valid(B1), ref.valid(B1)):
            assert torch.equal(x, y)
    if name == "c1":
        onbr, ogray, _, osrt = oracle.build_neighbors(rc.cpu().numpy())
        np.testing.assert_array_equal(a[0].cpu().numpy().view(np.uint32), onbr)
        np.testing.assert_array_equal(a[2].cpu().numpy(), osrt)
    g = torch.Generator(device=gpu)
    g.manual_seed(3)
    x = torch.randn((len(cc), 64), generator=g, device=gpu).to(torch.bfloat16)
    w = (torch.randn((64, 27, 64), generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    y1 = sp.subm_conv_fused(x, w, None, cache, act=sp.ACT_SILU, out_dtype=torch.float32)
    y2 = sp.subm_conv_fused(x, w, None, ref, act=sp.ACT_SILU, out_dtype=torch.float32)
    assert torch.equal(y1, y2)
    # no parents: empty level
    e_cc, e_src, e_cache = sp.subdivide_build(tc[:0], tl[:0])
    assert e_cc.shape == (0, 4) and e_src.shape == (0,) and e_cache.N == 0


def test_release_cached_memory(gpu):
    """Cached blocks go back to the driver: after a cache is dropped its buffers are cached; releasing them reports
    their bytes, the next build allocates from the driver again, and its map is unchanged."""
    import gc
    sp.set_stream(torch.cuda.current_stream())
    c = torch.from_numpy(W.shell_coords(W.CONFIGS["c1"])).to(gpu)
    a = sp.build_neighbors(c)
    ref = [t.clone() for t in a.tensors()]
    del a
    gc.collect()
    torch.cuda.synchronize()
    assert sp.release_cached_memory() > 0
    assert sp.release_cached_memory() == 0
    _, drv0 = sp.alloc_counts()
    b = sp.build_neighbors(c)
    _, drv1 = sp.alloc_counts()
    assert drv1 > drv0
    for x, y in zip(ref, b.tensors()):
        assert torch.equal(x, y)
