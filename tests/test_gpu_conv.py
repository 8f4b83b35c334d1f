"""GPU parity of the masked implicit-GEMM conv against the fp32 CPU oracle on the same (bf16/fp16-quantized)
inputs.

Every case runs the kernel twice: with an fp32 output and with the case's output dtype.
  * fp32 output vs the fp32 oracle: relative L2 <= 1e-5 and max-abs <= 1e-4 (well inside the stated bar of
    rel-L2 <= 1e-3, max-abs <= 2e-2); the two differ only in the order of the fp32 accumulation.
  * bf16/fp16 output: bit-identical to the fp32 output rounded (nearest-even) to that dtype -- the kernel rounds
    once, in the epilogue -- and within rel-L2 <= 1e-3 of the rounded oracle, each element within
    max(2e-2, one unit in the last place of the rounded oracle value). Rounding an fp32 result to bf16 alone costs
    ~1.7e-3 relative L2 on N(0,1) data, and two fp32 sums that differ in the last bit can round to neighbouring
    bf16 values (1 ulp = 0.03125 on [4, 8)), so the dtype comparison cannot be tighter than that.
"""
import dataclasses
import os

import numpy as np
import pytest
import torch

import oracle
import spconv_amd as sp
from spconv_amd import workloads as W

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def quantize(a, dt):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(TDT[dt])
    return t, t.float().numpy()


def ulp(a, dt):
    """Spacing of the bf16/fp16 grid at |a| (normal range)."""
    mant = 7 if dt == "bf16" else 10
    e = np.floor(np.log2(np.maximum(np.abs(a), 1e-30)))
    return np.exp2(e - mant)


def compare(y, ref, out_dt, what=""):
    yr = y.float().cpu().numpy()
    assert np.isfinite(yr).all(), what
    if out_dt != "f32":
        ref = torch.from_numpy(ref).to(TDT[out_dt]).float().numpy()
        tol = np.maximum(2e-2, ulp(ref, out_dt))
        rel_bar = 1e-3
    else:
        tol = np.full(ref.shape, 1e-4)
        rel_bar = 1e-5
    rel = np.linalg.norm(yr - ref) / max(np.linalg.norm(ref), 1e-30)
    err = np.abs(yr - ref)
    mx = err.max() if ref.size else 0.0
    assert rel <= rel_bar and np.all(err <= tol), f"{what}: rel-L2 {rel:.3g} max-abs {mx:.3g}"
    return rel, mx


def run_case(dev, c, ci, co, in_dt="bf16", out_dt="bf16", act=0, res_dt=None, bias_dt="f32", rows=None, seed=0,
             bounds=(4096, 4096, 4096)):
    n = len(c)
    print(f"conv case n={n} ci={ci} co={co} in={in_dt} out={out_dt} act={act} res={res_dt}", flush=True)
    cfg = W.Config("t", 0, 0, (0, 0), False, 0, ci, co, in_dt, "", 1000 + seed)
    w, b = W.conv_params(cfg)
    x = W.features(n, ci, seed + 1)
    tx, qx = quantize(x, in_dt)
    tw, qw = quantize(w, in_dt)
    tb, qb = quantize(b, bias_dt)
    tr = qr = None
    if res_dt:
        tr, qr = quantize(W.features(n, co, seed + 2), res_dt)
    tc = torch.from_numpy(c).to(dev)
    cache = sp.build_neighbors(tc, *bounds)
    args = (tx.to(dev), tw.to(dev), tb.to(dev), cache)
    rr = None if tr is None else tr.to(dev)
    y32 = sp.subm_conv_fused(*args, residual=rr, act=act, out_dtype=torch.float32)
    nbr, _, _, _ = oracle.build_neighbors(c, *bounds)
    ref = oracle.conv(qx, qw, qb, nbr, res=qr, act=act, rows=rows)
    sel = (lambda t: t) if rows is None else (lambda t: t[torch.from_numpy(np.asarray(rows)).to(dev)])
    what = f"n={n} ci={ci} co={co} {in_dt}->{out_dt} act={act} res={res_dt}"
    out = compare(sel(y32), ref, "f32", what)
    if out_dt != "f32":
        y = sp.subm_conv_fused(*args, residual=rr, act=act, out_dtype=TDT[out_dt])
        assert torch.equal(y, y32.to(TDT[out_dt])), what + ": low-precision output is not round(fp32 output)"
        out = compare(sel(y), ref, out_dt, what)
    return out


def shell(r, h=1.0, grid=None, seed=7):
    g = grid or int(2 * r + 6)
    return W.shell_coords(W.Config("s", g, 1, (r, r), False, h, 0, 0, "", "", seed, centred=True))


@pytest.mark.parametrize("ci,co", [(32, 64), (64, 64), (96, 64), (128, 64), (64, 128), (96, 128), (256, 256), (128, 192), (256, 512)])
def test_widths(gpu, ci, co):
    run_case(gpu, shell(9.0), ci, co, out_dt="bf16")


@pytest.mark.parametrize("in_dt", ["bf16", "f16"])
@pytest.mark.parametrize("act,res_dt", [(0, None), (1, None), (0, "bf16"), (1, "f32"), (0, "f16")])
def test_epilogues(gpu, in_dt, act, res_dt):
    run_case(gpu, shell(7.0), 64, 128, in_dt=in_dt, out_dt=in_dt, act=act, res_dt=res_dt)
    run_case(gpu, shell(7.0), 64, 64, in_dt=in_dt, out_dt=in_dt, act=act, res_dt=res_dt)


def test_reference_entry_point(gpu):
    """subm_conv (reference signature): output in x's dtype, fp16 bias like the decoder's weights."""
    c = shell(6.0)
    n = len(c)
    w, b = W.conv_params(W.CONFIGS["c5"], ci=64, co=64)
    x = W.features(n, 64, 3)
    tx, qx = quantize(x, "f16")
    tw, qw = quantize(w, "f16")
    tb, qb = quantize(b, "f16")
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    y = sp.subm_conv(tx.to(gpu), tw.to(gpu), tb.to(gpu), cache)
    assert y.dtype == torch.float16 and y.shape == (n, 64)
    nbr, _, _, _ = oracle.build_neighbors(c)
    compare(y, oracle.conv(qx, qw, qb, nbr), "f16")


def test_edges(gpu):
    # isolated voxels only (just the centre offset), tiles with one row, several batches, tight bounds
    c = np.array([[0, 0, 0, 0], [0, 3, 3, 3], [1, 0, 0, 0], [2, 7, 7, 7]], np.int32)
    run_case(gpu, c, 64, 64, out_dt="f32", bounds=(8, 8, 8))
    run_case(gpu, c, 256, 128, out_dt="f32", bounds=(8, 8, 8))
    # N not a multiple of the 128-row tile, one-voxel-wide lines, grid faces
    g = np.stack(np.meshgrid(np.arange(5), np.arange(5), np.arange(7), indexing="ij"), -1).reshape(-1, 3)
    c = np.concatenate([np.zeros((len(g), 1), np.int32), g.astype(np.int32)], 1)
    run_case(gpu, c, 64, 64, out_dt="f32", bounds=(5, 5, 7))
    # empty input
    cache = sp.build_neighbors(torch.zeros((0, 4), dtype=torch.int32, device=gpu))
    y = sp.subm_conv_fused(torch.zeros((0, 64), dtype=torch.bfloat16, device=gpu),
                           torch.zeros((64, 27, 64), dtype=torch.bfloat16, device=gpu), None, cache)
    assert y.shape == (0, 64)


def test_bad_arguments(gpu):
    c = shell(4.0)
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    n = len(c)
    x = torch.zeros((n, 48), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros((64, 27, 48), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        sp.subm_conv_fused(x, w, None, cache)
    x = torch.zeros((n + 1, 64), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros((64, 27, 64), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="rows"):
        sp.subm_conv_fused(x, w, None, cache)
    x = torch.zeros((n, 64), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="both"):
        sp.subm_conv_fused(x, w.half(), None, cache)


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_configs_all_rows(gpu, name):
    """Full-size workload on the GPU, every output row checked against the (multithreaded) oracle."""
    cfg = W.CONFIGS[name]
    c = W.shell_coords(cfg)
    act = 1 if "silu" in cfg.epilogue else 0
    res = "bf16" if "res" in cfg.epilogue else None
    run_case(gpu, c, cfg.ci, cfg.co, act=act, res_dt=res, seed=cfg.seed)


@pytest.mark.parametrize("r,co", [(40, 256), (45, 512), (65, 256), (60, 512)])
def test_wide_xcd_runs(gpu, r, co):
    """The longest-first schedule of the wide kernel dealt to the XCDs in runs of consecutive tiles, at tile counts
    whose last block of runs is partial in different ways (312, 798, 833 and 1416 tiles of 128 rows x 256 columns:
    remainders 56, 30, 65 and 8 of 128): every output row against the oracle, so a tile computed twice or never
    fails."""
    run_case(gpu, shell(r), 256, co, act=1, res_dt="bf16", seed=r)


def test_halo128_children(gpu, monkeypatch):
    """The halo kernel at Ci = 128 (opt-in, SPCONV_HALO128): two K chunks per offset, 128-row windows, spill tiles
    to the gathering kernel; c5-style children, every row against the oracle, plain and gathered."""
    monkeypatch.setenv("SPCONV_HALO128", "1")
    par = W.shell_coords(W.CONFIGS["c1"])
    lg = W.keep_logits(len(par), 0.5, 9)
    gc, _ = sp.subdivide(torch.from_numpy(par).to(gpu), torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16))
    c = gc.cpu().numpy()
    run_case(gpu, c, 128, 64, act=1, res_dt="bf16", seed=5)
    run_case(gpu, c, 128, 64, in_dt="f16", out_dt="f32", seed=6)


def test_c5_children(gpu):
    """C5's children (the subdivided 1024^3 level, 128 -> 64, bias + SiLU), every output row checked."""
    cfg = W.CONFIGS["c5"]
    par = W.shell_coords(cfg)
    tc = torch.from_numpy(par).to(gpu)
    lg = W.keep_logits(len(par), cfg.keep_frac, cfg.seed)
    gc, _ = sp.subdivide(tc, torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16))
    c = gc.cpu().numpy()
    run_case(gpu, c, cfg.ci, cfg.co, act=1, seed=cfg.seed)


def test_conv_golden_fixture(gpu):
    """Against tests/golden/small_shell.npz: y = silu(conv(x, w) + b) + r from float64 torch conv3d (Ci=32, Co=64)."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "small_shell.npz"))
    t = lambda k: torch.from_numpy(g[k]).to(gpu).view(torch.bfloat16)
    cache = sp.build_neighbors(torch.from_numpy(g["coords"]).to(gpu))
    y = sp.subm_conv_fused(t("x"), t("w"), t("b"), cache, residual=t("r"), act=sp.ACT_SILU, out_dtype=torch.float32)
    compare(y, g["y_silu_res"].astype(np.float32), "f32", "golden fixture")


# ------------------------------------------------------------------------------------------ gathered rows
@pytest.mark.parametrize("ci,co", [(128, 64), (64, 64), (32, 64), (256, 256), (64, 128)])
def test_gathered_conv(gpu, ci, co):
    """subm_conv_gathered on c2s children reading their parents' rows (row_map = src, shift 3) equals the conv of
    the materialized gathered rows bit for bit, and the fp32 oracle on them; map entries outside the source rows
    read zero rows."""
    par = W.shell_coords(W.CONFIGS["c1"])
    lg = W.keep_logits(len(par), 0.35, 3)
    ch, src = sp.subdivide(torch.from_numpy(par).to(gpu),
                           torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16))
    print(f"gathered case parents={len(par)} children={len(ch)} ci={ci} co={co}", flush=True)
    cache = sp.build_neighbors(ch.contiguous())
    cfg = W.Config("t", 0, 0, (0, 0), False, 0, ci, co, "bf16", "", 77)
    w, b = W.conv_params(cfg)
    tx, qx = quantize(W.features(len(par), ci, 5), "bf16")
    tw, qw = quantize(w, "bf16")
    tr, qr = quantize(W.features(len(ch), co, 6), "bf16")
    xs, ws, bs, rs = tx.to(gpu), tw.to(gpu), torch.from_numpy(b).to(gpu), tr.to(gpu)
    rmap = src.clone()
    rmap[::97] = (len(par) + 3) * 8  # past the source rows
    rmap[5::101] = -8                # negative
    for act in (0, 1):
        y1 = sp.subm_conv_gathered(xs, rmap, 3, ws, bs, cache, residual=rs, act=act, out_dtype=torch.float32)
        idx = rmap.long() >> 3
        ok = (idx >= 0) & (idx < len(par))
        xg = torch.zeros((len(ch), ci), dtype=torch.bfloat16, device=gpu)
        xg[ok] = xs[idx[ok]]
        y2 = sp.subm_conv_fused(xg, ws, bs, cache, residual=rs, act=act, out_dtype=torch.float32)
        assert torch.equal(y1, y2), f"ci={ci} co={co} act={act}: gathered != materialized"
        nbr, _, _, _ = oracle.build_neighbors(ch.cpu().numpy())
        ref = oracle.conv(xg.float().cpu().numpy(), qw, b, nbr, res=qr, act=act)
        compare(y1, ref, "f32", f"gathered ci={ci} co={co} act={act}")


@pytest.mark.parametrize("ci,co", [(128, 192), (96, 192), (64, 320), (64, 64), (128, 64), (64, 128), (256, 256),
                                   (768, 768)])
def test_f16_compat_epilogue(gpu, ci, co):
    """EPI_F16_COMPAT reproduces the reference's rounding sequence on the kernel's fp32 sums: f16(f16(acc) + b),
    then SiLU rounded to f16, then the residual add rounded to f16. Every kernel (generic, narrow, halo, wide) applies
    it in its epilogue, so the sequence applied on the host to the same kernel's fp32 output without bias is
    bit-exact without SiLU. With SiLU the host exp may differ from the device's in the last fp32 bit, so at most 1e-3
    of the elements may differ, by one fp16 ulp (plus, after a residual add, one ulp of the SiLU value that
    differed)."""
    c = shell(7.0) if ci < 768 else W.shell_coords(W.CONFIGS["c2"])[:3000]
    n = len(c)
    print(f"compat case n={n} ci={ci} co={co}", flush=True)
    w, b = W.conv_params(W.Config("t", 0, 0, (0, 0), False, 0, ci, co, "f16", "", 31))
    tx, _ = quantize(W.features(n, ci, 8), "f16")
    tw, _ = quantize(w, "f16")
    tb, _ = quantize(b * 10, "f16")
    tr, _ = quantize(W.features(n, co, 9), "f16")
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    xs, ws, bs, rs = tx.to(gpu), tw.to(gpu), tb.to(gpu), tr.to(gpu)
    acc = sp.subm_conv_fused(xs, ws, None, cache, out_dtype=torch.float32).cpu()
    for act in (0, 1):
        for res in (None, rs):
            y = sp.subm_conv_fused(xs, ws, bs, cache, residual=res, act=act | sp.EPI_F16_COMPAT).cpu()
            e = (acc.half().float() + tb.float()).half().float()
            if act:
                e = (e.double() / (1 + torch.exp(-e.double()))).float().half().float()
            s = e.clone()  # the SiLU value: a one-ulp difference there survives the residual add
            if res is not None:
                e = e + tr.float()
            e = e.half()
            what = f"ci={ci} co={co} act={act} res={res is not None}"
            assert y.dtype == torch.float16, what
            if not act:
                assert torch.equal(y, e), what
            else:
                d = (y.float() - e.float()).abs()
                bad = d > 0
                what += f": {int(bad.sum())} of {bad.numel()} differ, max {float(d.max()):.3g}"
                assert bad.float().mean() <= 1e-3, what
                tol = ulp(e.float()[bad].numpy(), "f16") + (ulp(s[bad].numpy(), "f16") if res is not None else 0)
                assert torch.all(d[bad] <= torch.from_numpy(tol)), what
    with pytest.raises(RuntimeError):  # bf16 is not a compat dtype
        sp.subm_conv_fused(xs.bfloat16(), ws.bfloat16(), None, cache, act=sp.EPI_F16_COMPAT)


def replay_reference(x, w, b, nbr, order, lst, seg, B1, BK, S, magnitude=False):
    """Host restatement of the split-K schedule for the test: fp64 partials per split over the split's K chunks of
    each B1 block (rounded to fp32, fp32 bias in split 0), then four interleaved fp32 accumulators, one fp16
    rounding. x [N,Ci], w [Co,27,Ci], b [Co] as float arrays of the fp16 inputs."""
    n, ci = x.shape
    co = w.shape[0]
    nk, cpv = ci // BK, ci // 32
    part = np.zeros((S, n, co), np.float64)
    xz = np.concatenate([x, np.zeros((1, ci))]).astype(np.float64)
    for blk in range(len(seg) - 1):
        rows = order[blk * B1:(blk + 1) * B1]
        vs, vl = seg[blk], seg[blk + 1] - seg[blk]
        for s in range(S):
            k0 = -(-nk * vl * s // S) * (BK // 32)
            k1 = -(-nk * vl * (s + 1) // S) * (BK // 32)
            for kc in range(k0, k1):
                v, c0 = lst[vs + kc // cpv], (kc % cpv) * 32
                src = nbr[rows, v].astype(np.int64)
                src[src == 0xFFFFFFFF] = n
                part[s, rows] += xz[src, c0:c0 + 32] @ w[:, v, c0:c0 + 32].astype(np.float64).T
    if magnitude:  # the fp64 sum of |terms| (x, w, b passed as absolute values): the scale of fp32 rounding errors
        return part.sum(0) + b
    part = part.astype(np.float32)
    part[0] += b.astype(np.float32)
    a = np.zeros((4, n, co), np.float32)
    for s in range(S):
        a[s & 3] = a[s & 3] + part[s]
    return (((a[0] + a[1]) + a[2]) + a[3]).astype(np.float16)


@pytest.mark.parametrize("ci,co,cfg", [(128, 64, (64, 32, 4)), (256, 128, (128, 64, 2)), (128, 96, (32, 32, 8)),
                                       (64, 64, (128, 64, 1))])
def test_replay_split_k(gpu, ci, co, cfg):
    """subm_conv_replay against the host restatement of the reference's split-K schedule and sum order: fp32 sums of
    one split may differ from the host's fp64-then-fp32 ones in the last bits (and the partials partly cancel), so at
    most 5e-3 of the elements may differ, by one fp16 ulp (the order itself is pinned by the known answer below); the whole output within the conv bar of the fp32 oracle. S == 1 equals the compat
    epilogue bit for bit."""
    c = shell(7.0)
    n = len(c)
    print(f"replay case n={n} ci={ci} co={co} cfg={cfg}", flush=True)
    w, b = W.conv_params(W.Config("t", 0, 0, (0, 0), False, 0, ci, co, "f16", "", 33))
    tx, qx = quantize(W.features(n, ci, 10), "f16")
    tw, qw = quantize(w, "f16")
    tb, qb = quantize(b * 10, "f16")
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    xs, ws, bs = tx.to(gpu), tw.to(gpu), tb.to(gpu)
    y = sp.subm_conv_replay(xs, ws, bs, cache, cfg)
    B1, BK, S = cfg
    nbr, gray, srt = cache.tensors()
    if S == 1:
        assert torch.equal(y, sp.subm_conv_fused(xs, ws, bs, cache, act=sp.EPI_F16_COMPAT))
    else:
        lst, seg = cache.valid(B1)
        args = (nbr.cpu().numpy().view(np.uint32), srt.cpu().numpy(), lst.cpu().numpy(), seg.cpu().numpy(), B1, BK, S)
        e = replay_reference(qx, qw, qb, *args)
        mag = replay_reference(np.abs(qx), np.abs(qw), np.abs(qb), *args, magnitude=True)
        d = np.abs(y.float().cpu().numpy() - e.astype(np.float32))
        bad = d > 0
        # one fp16 ulp of the result, plus the fp32 rounding of the partials (a few fp32 eps of the sum of |terms|,
        # which dominates where partials cancel to a result near zero)
        tol = ulp(e.astype(np.float32)[bad], "f16") + 2.0 ** -21 * mag[bad]
        assert bad.mean() <= 5e-3 and np.all(d[bad] <= tol), (int(bad.sum()), d.max())
    onbr, _, _, _ = oracle.build_neighbors(c)
    compare(y, oracle.conv(qx, qw, qb, onbr), "f16", f"replay {cfg}")
    # fused forms: SiLU then residual, each rounded to fp16 as the reference's separate passes
    tr, qr = quantize(W.features(n, co, 11), "f16")
    y2 = sp.subm_conv_replay(xs, ws, bs, cache, cfg, residual=tr.to(gpu), act=sp.ACT_SILU).float().cpu()
    yy = y.float().cpu().double()
    e2 = (yy / (1 + torch.exp(-yy))).float().half().float()
    e2 = (e2 + tr.float()).half().float()
    d = (y2 - e2).abs()
    bad = d > 0
    assert bad.float().mean() <= 5e-3


def test_replay_empty_null_buffers(gpu):
    """spc_subm_conv_replay on an empty cache accepts null buffers like its sibling entry points (N == 0: nothing is
    read or written); a nonempty call with a null buffer is an error."""
    import ctypes
    lib = sp.load_library()
    cache = sp.build_neighbors(torch.zeros((0, 4), dtype=torch.int32, device=gpu))
    assert lib.spc_subm_conv_replay(None, None, None, None, 0, 0, 64, 64, 128, 64, 1, cache._h, None) == 0, \
        lib.spc_last_error()
    c = shell(3.0)
    full = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    assert lib.spc_subm_conv_replay(None, None, None, None, 0, len(c), 64, 64, 128, 64, 1, full._h, None) == -1
    assert b"null argument" in lib.spc_last_error()


def test_replay_split_order_known_answer(gpu):
    """One isolated voxel, Ci = 256, BK = 32, S = 8: split s holds exactly the 32-channel chunk s of the centre offset.
    The weights make chunk s's partial p_s = (32768, 2^-9, 0, 0, -32768, 2^-9, 0, 0) for output channel 0, and the
    fp16 bias 2^-9 joins split 0 in fp32 (32768 + 2^-9 rounds back to 32768). Four interleaved accumulators give
    a0 = p0 + p4 = 0 and a1 = p1 + p5 = 2^-8, so y = 2^-8; a left-to-right sum of the splits would give 2^-9, and
    an fp16 bias add after the rounding 2^-8 + 2^-9."""
    c = np.array([[0, 5, 5, 5]], np.int32)
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    x = torch.zeros((1, 256), dtype=torch.float16)
    x[0, ::32] = 1.0
    w = torch.zeros((64, 27, 256), dtype=torch.float16)
    p = [32768.0, 2.0 ** -9, 0.0, 0.0, -32768.0, 2.0 ** -9, 0.0, 0.0]
    for j, v in enumerate(p):
        w[:, 13, 32 * j] = v
    b = torch.full((64,), 2.0 ** -9, dtype=torch.float16)
    y = sp.subm_conv_replay(x.to(gpu), w.to(gpu), b.to(gpu), cache, (128, 32, 8)).cpu()
    assert torch.all(y == 2.0 ** -8), y[0, :4]


def test_halo_fallback_shuffled_rows(gpu):
    """64 -> 64 on a shell whose rows are shuffled: every 256-row window then reads far more than 512 distinct
    neighbour rows, so every tile is a spill tile and the gathering kernel computes all rows -- same results
    either way (checked against the oracle); the unshuffled shell takes the halo kernel."""
    c = shell(12.0)
    rng = np.random.default_rng(4)
    shuffled = c[rng.permutation(len(c))]
    for coords in (c, shuffled):
        run_case(gpu, coords, 64, 64, res_dt="bf16")


def mixed_spill_coords():
    """A sparse sphere shell plus a dense 12^3 block, Morton-sorted: the block's 256-row windows are 8x8x4 bricks
    whose 10x10x6 halos (600 rows) exceed the 512-row LDS halo, so those tiles spill to the gathering kernel while
    the shell's tiles stay on the halo kernel."""
    s = shell(10.0, grid=26)
    g = np.stack(np.meshgrid(*(np.arange(30, 42),) * 3, indexing="ij"), -1).reshape(-1, 3)
    p = np.concatenate([s[:, 1:], g]).astype(np.int64)
    p = p[np.argsort(W.morton3(p[:, 0], p[:, 1], p[:, 2]), kind="stable")]
    return np.concatenate([np.zeros((len(p), 1), np.int64), p], 1).astype(np.int32)


def test_halo_spill_tiles(gpu):
    """Spill tiles of the halo schedule run on the gathering kernel, the rest on the halo kernel: every row checked
    against the oracle, with and without SiLU / residual, and the tail tile partial."""
    c = mixed_spill_coords()
    run_case(gpu, c, 64, 64, res_dt="bf16")
    run_case(gpu, c, 64, 64, act=1, out_dt="f32")
    run_case(gpu, c[:4092], 64, 64, res_dt="bf16", seed=3)  # the last tile partial (252 rows) and a spill tile


def test_halo_spill_gathered_and_skip(gpu):
    """Gathered conv (row map) and the upsample skip on a cache with spill tiles: the gathered conv equals the conv
    of the materialized rows bit for bit (the spill tiles read their rows through the map too), and the skip
    variant (the halo kernel, and the gathering kernel on the spill tiles, each adding the skip rows in its epilogue)
    equals the conv with the materialized skip rows as its residual bit for bit, and conv + add_skip (two roundings)
    within rel-L2 2e-3."""
    c = mixed_spill_coords()
    n = len(c)
    m = n // 2 + 5
    g = torch.Generator().manual_seed(5)
    xs = torch.randn((m, 64), generator=g).to(torch.bfloat16).to(gpu)
    rmap = torch.randint(-8, 8 * m + 40, (n,), generator=g, dtype=torch.int32).to(gpu)
    w, b = W.conv_params(W.Config("t", 0, 0, (0, 0), False, 0, 64, 64, "bf16", "", 51))
    ws, bs = torch.from_numpy(w).to(torch.bfloat16).to(gpu), torch.from_numpy(b).to(gpu)
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    y1 = sp.subm_conv_gathered(xs, rmap, 3, ws, bs, cache, act=1, out_dtype=torch.float32)
    idx = rmap.long() >> 3
    ok = (idx >= 0) & (idx < m)
    xg = torch.zeros((n, 64), dtype=torch.bfloat16, device=gpu)
    xg[ok] = xs[idx[ok]]
    y2 = sp.subm_conv_fused(xg, ws, bs, cache, act=1, out_dtype=torch.float32)
    assert torch.equal(y1, y2), "gathered != materialized on a cache with spill tiles"
    nbr, _, _, _ = oracle.build_neighbors(c)
    wq = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
    compare(y1, oracle.conv(xg.float().cpu().numpy(), wq, b, nbr, act=1), "f32", "spill gathered")
    src = torch.randint(0, 8 * m, (n,), generator=g, dtype=torch.int32).to(gpu)
    y3 = sp.subm_conv_skip(xg, ws, bs, cache, xs, src, act=1)
    sl = src.long()
    cols = (sl[:, None] & 7) * 8 + torch.arange(64, device=gpu)[None, :] // 8  # Cin = 64: rep = 64 / 8 = 8
    skip_rows = xs[(sl >> 3)[:, None], cols]
    y5 = sp.subm_conv_fused(xg, ws, bs, cache, residual=skip_rows, act=1)
    if not os.environ.get("SPCONV_NO_HALO"):  # without the halo kernel the skip is a separate pass (two roundings)
        assert torch.equal(y3, y5), "skip variant != conv with the skip rows as residual on a cache with spill tiles"
    y4 = sp.subm_conv_fused(xg, ws, bs, cache, act=1)
    sp.add_skip(y4, xs, src)
    rel = ((y3.float() - y4.float()).norm() / y4.float().norm()).item()
    assert rel <= 2e-3, f"fused skip vs conv + add_skip: rel-L2 {rel:.3g}"


@pytest.mark.parametrize("nrows", [25309, 22000, 23800, 10842, 3000, 700])
def test_wide_tail_split(gpu, nrows, monkeypatch):
    """768 -> 768 (C2 coordinates, first nrows rows): 3 x ceil(nrows/128) tiles put 65-75 tiles on each XCD, more
    than its 64 concurrent workgroups, so the wide kernel splits each XCD's last tiles over several workgroups along
    K and reduces their fp32 partials; at 10842 / 3000 / 700 rows (32, 9, 2-3 tiles per XCD) every tile is split,
    over 2, 7 and 8 workgroups. Split and unsplit schedules differ only in the fp32 summation order: fp32
    outputs within rel-L2 1e-6, bf16 outputs within one bf16 ulp (+1e-5 absolute); every row of the split result
    is checked against the oracle. The coordinates are C2's spheres with a thicker shell (h = 2.35, 25 309 rows),
    so that the row-tile counts reach the split range."""
    cfg = dataclasses.replace(W.CONFIGS["c2"], half_thickness=2.35)
    c = W.shell_coords(cfg)[:nrows]
    n = len(c)
    print(f"tail split case n={n}", flush=True)
    w, b = W.conv_params(cfg)
    tx, qx = quantize(W.features(n, cfg.ci, 11), "bf16")
    tw, qw = quantize(w, "bf16")
    tb, qb = quantize(b, "f32")
    tr, qr = quantize(W.features(n, cfg.co, 12), "bf16")
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    args = (tx.to(gpu), tw.to(gpu), tb.to(gpu), cache)
    rr = tr.to(gpu)
    outs = {}
    for split in (True, False):
        if split:
            monkeypatch.delenv("SPCONV_NO_SPLIT", raising=False)
        else:
            monkeypatch.setenv("SPCONV_NO_SPLIT", "1")
        outs[split] = (sp.subm_conv_fused(*args, residual=rr, act=0, out_dtype=torch.float32),
                       sp.subm_conv_fused(*args, residual=rr, act=0, out_dtype=torch.bfloat16))
    monkeypatch.delenv("SPCONV_NO_SPLIT", raising=False)
    (s32, s16), (u32, u16) = outs[True], outs[False]
    rel = (torch.linalg.norm(s32 - u32) / torch.linalg.norm(u32)).item()
    assert rel <= 1e-6, f"split vs unsplit fp32 rel-L2 {rel:.3g}"
    assert torch.equal(s16, s32.to(torch.bfloat16)), "bf16 output is not round(fp32 output)"
    d16 = (s16.float() - u16.float()).abs()
    # one bf16 ulp of the value, plus 1e-5 absolute: near zero the fp32 reordering difference (~1e-6 of the partial
    # sums' magnitude) exceeds the ulp of a tiny result
    tol16 = torch.from_numpy(ulp(u16.float().cpu().numpy(), "bf16")).to(gpu) + 1e-5
    assert torch.all(d16 <= tol16), f"split vs unsplit bf16: max diff {d16.max().item():.3g}"
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert not torch.equal(s32, u32), "expected the split schedule on a 256-CU part"
    nbr, _, _, _ = oracle.build_neighbors(c)
    ref = oracle.conv(qx, qw, qb, nbr, res=qr, act=0)
    compare(s32, ref, "f32", f"split n={n}")


def test_wide_tail_split_256_f16(gpu, monkeypatch):
    """256 -> 256, fp16, bias + SiLU on the first 80000 rows of the C3 shell: 625 single-channel-tile row tiles,
    79 per XCD (72 on the last), so the last 15 (8) tiles of each XCD are split along K over 4 (8) workgroups on a
    256-CU part. Split vs unsplit fp32 outputs within
    rel-L2 1e-6; every row of the split result against the oracle."""
    c = W.shell_coords(W.CONFIGS["c3"])[:80000]
    n = len(c)
    print(f"tail split case n={n} 256->256 f16", flush=True)
    cfg = W.Config("t", 0, 0, (0, 0), False, 0, 256, 256, "f16", "", 31)
    w, b = W.conv_params(cfg)
    tx, qx = quantize(W.features(n, 256, 13), "f16")
    tw, qw = quantize(w, "f16")
    tb, qb = quantize(b, "f32")
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    args = (tx.to(gpu), tw.to(gpu), tb.to(gpu), cache)
    monkeypatch.setenv("SPCONV_NO_SPLIT", "1")
    u32 = sp.subm_conv_fused(*args, act=1, out_dtype=torch.float32)
    monkeypatch.delenv("SPCONV_NO_SPLIT", raising=False)
    s32 = sp.subm_conv_fused(*args, act=1, out_dtype=torch.float32)
    s16 = sp.subm_conv_fused(*args, act=1, out_dtype=torch.float16)
    rel = (torch.linalg.norm(s32 - u32) / torch.linalg.norm(u32)).item()
    assert rel <= 1e-6, f"split vs unsplit fp32 rel-L2 {rel:.3g}"
    assert torch.equal(s16, s32.to(torch.float16)), "fp16 output is not round(fp32 output)"
    nbr, _, _, _ = oracle.build_neighbors(c)
    ref = oracle.conv(qx, qw, qb, nbr, act=1)
    compare(s32, ref, "f32", f"split 256 n={n}")


def split_vs_unsplit(gpu, monkeypatch, c, ci, co, dt, act, res_dt, seed, w256=True):
    """Runs the conv with and without K splitting (SPCONV_NO_SPLIT), checks the two fp32 outputs agree to the fp32
    summation order (rel-L2 1e-6), the 16-bit output is round(fp32), and every row of the split result against the
    oracle. Returns whether the two schedules differed at all (they do when a split happened)."""
    if w256:
        monkeypatch.setenv("SPCONV_W256", "1")
    n = len(c)
    cfg = W.Config("t", 0, 0, (0, 0), False, 0, ci, co, dt, "", seed)
    w, b = W.conv_params(cfg)
    tx, qx = quantize(W.features(n, ci, seed + 1), dt)
    tw, qw = quantize(w, dt)
    tb, qb = quantize(b, "f32")
    tr = qr = None
    if res_dt:
        tr, qr = quantize(W.features(n, co, seed + 2), res_dt)
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    args = (tx.to(gpu), tw.to(gpu), tb.to(gpu), cache)
    rr = None if tr is None else tr.to(gpu)
    monkeypatch.setenv("SPCONV_NO_SPLIT", "1")
    u32 = sp.subm_conv_fused(*args, residual=rr, act=act, out_dtype=torch.float32)
    monkeypatch.delenv("SPCONV_NO_SPLIT", raising=False)
    s32 = sp.subm_conv_fused(*args, residual=rr, act=act, out_dtype=torch.float32)
    s16 = sp.subm_conv_fused(*args, residual=rr, act=act, out_dtype=TDT[dt])
    rel = (torch.linalg.norm(s32 - u32) / torch.linalg.norm(u32)).item()
    assert rel <= 1e-6, f"split vs unsplit fp32 rel-L2 {rel:.3g}"
    assert torch.equal(s16, s32.to(TDT[dt])), "16-bit output is not round(fp32 output)"
    nbr, _, _, _ = oracle.build_neighbors(c)
    ref = oracle.conv(qx, qw, qb, nbr, res=qr, act=act)
    compare(s32, ref, "f32", f"split n={n} {ci}->{co}")
    return not torch.equal(s32, u32)


@pytest.mark.parametrize("nrows", [10842, 6000, 2000])
def test_w256_k_split(gpu, monkeypatch, nrows):
    """256 x 256 tile kernel (SPCONV_W256=1), 768 -> 768 bf16 with bias + residual on C2's shell (its first nrows
    rows): 3 x ceil(nrows/256) tiles do not fill 256 CUs, so each tile's K stages are split over several workgroups and their fp32
    partials summed by k_split_reduce256."""
    c = W.shell_coords(W.CONFIGS["c2"])[:nrows]
    print(f"w256 split case n={len(c)}", flush=True)
    differed = split_vs_unsplit(gpu, monkeypatch, c, 768, 768, "bf16", 0, "bf16", 41)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert differed, "expected a K split on a 256-CU part"


def test_w256_k_split_f16_silu(gpu, monkeypatch):
    """256 x 256 tile kernel, 256 -> 512 fp16 with SiLU on the first 9000 rows of the C3 shell (36 x 2 tiles): K
    split, two column tiles."""
    c = W.shell_coords(W.CONFIGS["c3"])[:9000]
    print(f"w256 split case n={len(c)} 256->512 f16", flush=True)
    split_vs_unsplit(gpu, monkeypatch, c, 256, 512, "f16", 1, None, 43)


def test_c3_w256_kernel(gpu, monkeypatch):
    """The 256 x 256 tile kernel (SPCONV_W256=1) on the full C3 workload, every row against the oracle."""
    monkeypatch.setenv("SPCONV_W256", "1")
    cfg = W.CONFIGS["c3"]
    run_case(gpu, W.shell_coords(cfg), cfg.ci, cfg.co, act=1, seed=cfg.seed)


@pytest.mark.parametrize("ci,co", [(256, 256), (64, 256), (128, 768)])
def test_w256_widths(gpu, monkeypatch, ci, co):
    """256 x 256 tile kernel on a small shell (few tiles: K split) and every epilogue."""
    monkeypatch.setenv("SPCONV_W256", "1")
    c = shell(10.0)
    run_case(gpu, c, ci, co, act=1, res_dt="bf16", seed=3)
    run_case(gpu, c, ci, co, in_dt="f16", out_dt="f16", act=0, res_dt="f32", seed=4)


def test_c3_w8_kernel(gpu, monkeypatch):
    """The 8-wavefront 256 x 256 kernel with both operands in LDS (SPCONV_W8=1) on the full C3 workload, every row
    against the oracle."""
    monkeypatch.setenv("SPCONV_W8", "1")
    cfg = W.CONFIGS["c3"]
    run_case(gpu, W.shell_coords(cfg), cfg.ci, cfg.co, act=1, seed=cfg.seed)


@pytest.mark.parametrize("ci,co", [(256, 256), (32, 256), (96, 512), (768, 768)])
def test_w8_widths(gpu, monkeypatch, ci, co):
    """8-wavefront 256 x 256 kernel on a small shell (ragged last tile) and every epilogue."""
    monkeypatch.setenv("SPCONV_W8", "1")
    c = shell(10.0)
    run_case(gpu, c, ci, co, act=1, res_dt="bf16", seed=3)
    run_case(gpu, c, ci, co, in_dt="f16", out_dt="f16", act=0, res_dt="f32", seed=4)


def test_c5_gathered_full(gpu):
    """The timed cascade upsample path at C5's full size: subdivide_build on the 0.8 M parents, then
    subm_conv_gathered(x_parents, src, 3) 128 -> 64 with bias + SiLU on the fresh children's cache; every child row
    against the fp32 oracle on the gathered rows x_parents[src >> 3] (reference k_gather_rows + subm_conv,
    src/sdec.cu:34-43,70-87), fp32 and bf16 outputs."""
    cfg = W.CONFIGS["c5"]
    par = W.shell_coords(cfg)
    lg = W.keep_logits(len(par), cfg.keep_frac, cfg.seed)
    ch, src, cc = sp.subdivide_build(torch.from_numpy(par).to(gpu),
                                     torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16))
    n = len(ch)
    print(f"c5 gathered full: parents={len(par)} children={n}", flush=True)
    w, b = W.conv_params(cfg)
    tx, qx = quantize(W.features(len(par), cfg.ci, 21), "bf16")
    tw, qw = quantize(w, "bf16")
    xs, ws, bs = tx.to(gpu), tw.to(gpu), torch.from_numpy(b).to(gpu)
    y32 = sp.subm_conv_gathered(xs, src, 3, ws, bs, cc, act=1, out_dtype=torch.float32)
    y16 = sp.subm_conv_gathered(xs, src, 3, ws, bs, cc, act=1)
    assert torch.equal(y16, y32.to(torch.bfloat16)), "bf16 output is not round(fp32 output)"
    xg = qx[src.long().cpu().numpy() >> 3]
    nbr, _, _, _ = oracle.build_neighbors(ch.cpu().numpy())
    ref = oracle.conv(xg, qw, b, nbr, act=1)
    compare(y32, ref, "f32", "c5 gathered fp32")
    compare(y16, ref, "bf16", "c5 gathered bf16")


def test_c5_conv_skip_full(gpu):
    """subm_conv_skip (conv2 64 -> 64 + bias + SiLU with the c2s skip fused into the epilogue) on C5's children at
    full size: every row against the fp32 oracle with the skip rows repeat_interleave(C2S(x_parents)) as its
    residual (reference conv2 + k_add_skip, src/sdec.cu:38-43,82-84). The fused form rounds once; conv + add_skip
    rounds twice, so the two are compared to the oracle separately."""
    cfg = W.CONFIGS["c5"]
    par = W.shell_coords(cfg)
    lg = W.keep_logits(len(par), cfg.keep_frac, cfg.seed)
    ch, src, cc = sp.subdivide_build(torch.from_numpy(par).to(gpu),
                                     torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16))
    n, cin, co = len(ch), cfg.ci, 64
    print(f"c5 conv skip full: children={n}", flush=True)
    w, b = W.conv_params(W.Config("t", 0, 0, (0, 0), False, 0, co, co, "bf16", "", 61))
    th, qh = quantize(W.features(n, co, 22), "bf16")
    tp, qp = quantize(W.features(len(par), cin, 23), "bf16")
    tw, qw = quantize(w, "bf16")
    h, xp, ws, bs = th.to(gpu), tp.to(gpu), tw.to(gpu), torch.from_numpy(b).to(gpu)
    y = sp.subm_conv_skip(h, ws, bs, cc, xp, src, act=1)
    y2 = sp.subm_conv_fused(h, ws, bs, cc, act=1)
    sp.add_skip(y2, xp, src)
    s = src.long().cpu().numpy()
    rep = co // (cin // 8)
    cols = (s[:, None] & 7) * (cin // 8) + np.arange(co)[None, :] // rep
    skip = qp[(s >> 3)[:, None], cols]
    nbr, _, _, _ = oracle.build_neighbors(ch.cpu().numpy())
    ref = oracle.conv(qh, qw, b, nbr, res=skip, act=1)
    yr, y2r = y.float().cpu().numpy(), y2.float().cpu().numpy()
    rel2 = np.linalg.norm(y2r - ref) / np.linalg.norm(ref)
    assert rel2 <= 2e-3 and np.all(np.abs(y2r - ref) <= np.maximum(2e-2, 2 * ulp(ref, "bf16"))), \
        f"conv + add_skip: rel-L2 {rel2:.3g}"
    if os.environ.get("SPCONV_NO_HALO", "0") not in ("", "0"):
        # without the halo kernel subm_conv_skip is the conv, then add_skip: the same two roundings as y2
        assert torch.equal(y, y2), "subm_conv_skip without the halo kernel is conv + add_skip"
        return
    compare(y, ref, "bf16", "c5 conv skip (fused)")
    assert np.linalg.norm(yr - ref) <= np.linalg.norm(y2r - ref) * 1.01, "one rounding should not be worse than two"


def test_kernel_timing(gpu):
    """spc_kernel_timing brackets each conv call's conv kernels with events: one time per call, positive, below the
    host-timed call including the weight repack; off again, calls add no records."""
    import time
    c = shell(10.0)
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    x = torch.randn((len(c), 256), device=gpu).to(torch.bfloat16)
    w = (torch.randn((256, 27, 256), device=gpu) / 83).to(torch.bfloat16)
    y = sp.subm_conv_fused(x, w, None, cache)
    torch.cuda.synchronize()
    sp.kernel_timing(True)
    t0 = time.perf_counter()
    for _ in range(3):
        sp.subm_conv_fused(x, w, None, cache, out=y)
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3
    sp.kernel_timing(False)
    sp.subm_conv_fused(x, w, None, cache, out=y)
    t = sp.kernel_times()
    assert len(t) == 3 and all(v > 0 for v in t) and sum(t) <= host_ms, (t, host_ms)


@pytest.mark.parametrize("ci,co,r", [(1024, 1024, 6.0), (1024, 4096, 5.0), (512, 512, 8.0), (512, 2048, 7.0),
                                     (256, 1024, 9.0), (128, 128, 12.0), (128, 512, 11.0)])
def test_decoder_level_widths(gpu, ci, co, r):
    """The sparse decoders' layer widths (C = 1024 -> 512 -> 256 -> 128 -> 64; ConvNeXt convs C -> C and up-convs
    C -> 8 * C/2, as the reference's autotune keys list them, e.g. (2^11, 1024, 4096, 27)), on small shells: fp32
    output against the oracle, bf16 output = round(fp32 output). These shapes take the wide kernels' split schedules
    (few rows, many channels)."""
    run_case(gpu, shell(r), ci, co, act=1, res_dt="bf16", seed=int(r))
