"""Writes tests/golden/small_shell.npz: a small known-answer fixture computed WITHOUT the oracle.

Kernel map: brute-force dictionary lookups over the 27 offsets (v <-> (v/9-1, v/3%3-1, v%3-1), EMPTY =
0xffffffff), the neighbour mask from the map, the decoded mask as the xor of shifted masks, the row order by
Python's stable sorted(), and valid(B1) lists by a per-block OR. Conv: float64 torch.nn.functional.conv3d on the
dense grid the sparse set is scattered into (submanifold conv = zero-padded dense conv sampled at active sites),
plus bias, SiLU and a residual. Inputs are stored as bf16 bit patterns, so CPU and GPU read identical values.

usage: python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
EMPTY = 0xFFFFFFFF


def coords():
    """Two batches: a sphere shell (r=3.5) and a small tilted slab, ~300 voxels, shuffled row order."""
    pts = []
    g = np.stack(np.meshgrid(np.arange(12), np.arange(12), np.arange(12), indexing="ij"), -1).reshape(-1, 3)
    d = np.sqrt(((g - 5.5) ** 2).sum(1))
    for p in g[np.abs(d - 3.5) <= 0.7]:
        pts.append((0, *p))
    for p in g:
        if 2 <= p[0] <= 9 and 3 <= p[1] <= 8 and abs(p[2] - (p[0] // 2 + 2)) <= 0:
            pts.append((1, *p))
    c = np.array(pts, np.int32)
    return c[np.random.default_rng(7).permutation(len(c))]


def kernel_map(c):
    idx = {tuple(r): i for i, r in enumerate(c.tolist())}
    n = len(c)
    nbr = np.full((n, 27), EMPTY, np.uint32)
    for i, (b, x, y, z) in enumerate(c.tolist()):
        for v in range(27):
            j = idx.get((b, x + v // 9 - 1, y + v // 3 % 3 - 1, z + v % 3 - 1))
            if j is not None:
                nbr[i, v] = j
    gray = [sum(1 << v for v in range(27) if nbr[i, v] != EMPTY) for i in range(n)]
    dec = []
    for g in gray:
        b = 0
        for k in range(27):
            b ^= g >> k
        dec.append(b)
    order = sorted(range(n), key=lambda i: dec[i])
    return nbr, np.array(gray, np.int32), np.array(dec, np.int32), np.array(order, np.int32)


def valid(gray, order, B1):
    lst, seg = [], [0]
    for s in range(0, len(order), B1):
        o = 0
        for i in order[s:s + B1]:
            o |= int(gray[i])
        lst += [v for v in range(27) if o >> v & 1]
        seg.append(len(lst))
    return np.array(lst, np.int32), np.array(seg, np.int32)


def bf16_exact(a):
    return torch.from_numpy(a).to(torch.bfloat16).to(torch.float64).numpy()


def conv(c, ci, co, seed):
    rng = np.random.default_rng(seed)
    n = len(c)
    x = bf16_exact(rng.standard_normal((n, ci)))
    w = bf16_exact(rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci))
    b = bf16_exact(rng.standard_normal(co) * 0.1)
    r = bf16_exact(rng.standard_normal((n, co)))
    nb = int(c[:, 0].max()) + 1
    G = int(c[:, 1:].max()) + 1
    X = torch.zeros((nb, ci, G, G, G), dtype=torch.float64)
    X[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]] = torch.from_numpy(x)
    Wt = torch.from_numpy(w).reshape(co, 3, 3, 3, ci).permute(0, 4, 1, 2, 3).contiguous()
    Y = torch.nn.functional.conv3d(X, Wt, torch.from_numpy(b), padding=1)
    y = Y[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]].numpy()
    y_silu_res = y / (1.0 + np.exp(-y)) + r
    bits = lambda a: torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy()  # exact: a is bf16-valued
    return bits(x), bits(w), bits(b), bits(r), y_silu_res.astype(np.float32)


def main():
    c = coords()
    nbr, gray, dec, order = kernel_map(c)
    l32, s32 = valid(gray, order, 32)
    l128, s128 = valid(gray, order, 128)
    x, w, b, r, ysr = conv(c, 32, 64, 11)
    # x, w, b, r: bf16 bit patterns (int16); y_silu_res = silu(conv(x, w) + b) + r in float32
    np.savez_compressed(os.path.join(HERE, "small_shell.npz"), coords=c, nbr=nbr, gray=gray, dec=dec, order=order,
                        list32=l32, seg32=s32, list128=l128, seg128=s128, x=x, w=w, b=b, r=r, y_silu_res=ysr)
    print("wrote", len(c), "voxels")


if __name__ == "__main__":
    main()
