"""GPU parity of the one-pass (gather +) LayerNorm + SiLU pre-activation against torch's fp32 layer_norm / silu on
the same (bf16/fp16) inputs, gathered on the host.

The kernel rounds once, from fp32, so each element is within one unit in the last place of the fp32 reference
rounded to the dtype (two fp32 values differing in the last bits can round to neighbouring grid points) and the
relative L2 error is that of one rounding: <= 1e-3 for fp16 and <= 3e-3 for bf16 (one bf16 rounding alone costs
~1.7e-3 on N(0,1) data). Rows whose map entry points outside the source are LN(0) = beta.
"""
import numpy as np
import pytest
import torch

import spconv_amd as sp

pytestmark = pytest.mark.gpu


def ulp(a, dt):
    mant = 7 if dt == torch.bfloat16 else 10
    e = np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** -14)))
    return np.exp2(e - mant)


def reference(x_src, rmap, shift, gamma, beta, eps, act):
    x = x_src.float().cpu()
    if rmap is not None:
        idx = rmap.cpu().long() >> shift
        ok = (idx >= 0) & (idx < len(x))
        xg = torch.zeros((len(idx), x.shape[1]))
        xg[ok] = x[idx[ok]]
        x = xg
    y = torch.nn.functional.layer_norm(x, (x.shape[1],), None if gamma is None else gamma.cpu(),
                                       None if beta is None else beta.cpu(), eps)
    return torch.nn.functional.silu(y) if act else y


def check(y, ref, dt, what):
    r = ref.to(dt).float().numpy()
    yr = y.float().cpu().numpy()
    assert np.isfinite(yr).all(), what
    err = np.abs(yr - r)
    rel = np.linalg.norm(yr - ref.numpy()) / max(np.linalg.norm(ref.numpy()), 1e-30)
    bar = 3e-3 if dt == torch.bfloat16 else 1e-3
    assert np.all(err <= ulp(r, dt) + 1e-6) and rel <= bar, f"{what}: max-abs {err.max():.3g} rel-L2 {rel:.3g}"


@pytest.mark.parametrize("C", [8, 32, 64, 128, 256, 1024, 4096])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_ln_act_identity(gpu, C, dt):
    """LayerNorm(x) * gamma + beta then SiLU, rows in order (an upsample block's first pre-activation)."""
    print(f"ln case C={C} dt={dt}", flush=True)
    g = torch.Generator().manual_seed(C)
    n = 3001 if C <= 1024 else 300
    x = (torch.randn((n, C), generator=g) * 2 + 0.5).to(dt)
    x[7] = 3.0  # a constant row: variance 0
    x[8] += 60.0  # a large mean
    gamma = torch.rand(C, generator=g) + 0.5
    beta = torch.randn(C, generator=g) * 0.1
    for affine in (False, True):
        for act in (0, 1):
            gm, bt = (gamma.to(gpu), beta.to(gpu)) if affine else (None, None)
            y = sp.gather_ln_act(x.to(gpu), gamma=gm, beta=bt, eps=1e-6, act=act)
            check(y, reference(x, None, 0, gm, bt, 1e-6, act), dt, f"C={C} affine={affine} act={act}")


@pytest.mark.parametrize("C", [16, 64, 128, 512])
def test_gather_ln_act(gpu, C):
    """Children reading their parents' rows (row_map = c2s src, shift 3), with entries outside the source."""
    print(f"gather-ln case C={C}", flush=True)
    g = torch.Generator().manual_seed(100 + C)
    M = 1500
    x = torch.randn((M, C), generator=g).to(torch.bfloat16)
    rmap = torch.randint(0, M * 8, (9000,), generator=g, dtype=torch.int32)
    rmap[::97] = (M + 3) * 8
    rmap[5::101] = -8
    beta = torch.randn(C, generator=g)
    for bt in (None, beta):
        y = sp.gather_ln_act(x.to(gpu), rmap.to(gpu), 3, beta=None if bt is None else bt.to(gpu), act=1)
        check(y, reference(x, rmap, 3, None, bt, 1e-6, 1), torch.bfloat16, f"C={C} beta={bt is not None}")


def test_gather_ln_act_empty_and_errors(gpu):
    x = torch.randn((10, 64), device=gpu).to(torch.bfloat16)
    y = sp.gather_ln_act(x, torch.zeros(0, dtype=torch.int32, device=gpu), 3)
    assert y.shape == (0, 64)
    with pytest.raises(RuntimeError):
        sp.gather_ln_act(torch.randn((10, 48), device=gpu).to(torch.bfloat16))  # C/8 = 6: not a power of two
    with pytest.raises(RuntimeError):
        sp.gather_ln_act(x.float())  # fp32 input


def skip_reference(h, x, src):
    """h + repeat_interleave(C2S(x), rep, dim=1): the c2s view of x is x.view(8n, Cin/8), row src[i]."""
    n, Cin = x.shape
    Cs = Cin // 8
    rep = h.shape[1] // Cs
    xs = x.reshape(n * 8, Cs)[src.long()].repeat_interleave(rep, dim=1)
    return (h.float() + xs.float()).to(h.dtype)


@pytest.mark.parametrize("Cin,Co", [(64, 8), (512, 64), (256, 64), (128, 64), (1024, 256), (64, 64)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_add_skip(gpu, Cin, Co, dt):
    """Bit-identical to the fp32 sum rounded once (the reference's arithmetic), for rep = 1, 2, 4, 8 and 64."""
    print(f"add_skip case Cin={Cin} Co={Co} dt={dt}", flush=True)
    g = torch.Generator().manual_seed(Cin + Co)
    n, m = 700, 2100
    x = torch.randn((n, Cin), generator=g).to(dt)
    src = torch.randint(0, n * 8, (m,), generator=g, dtype=torch.int32)
    h = torch.randn((m, Co), generator=g).to(dt)
    hg = h.to(gpu)
    sp.add_skip(hg, x.to(gpu), src.to(gpu))
    assert torch.equal(hg.cpu(), skip_reference(h, x, src))


def test_add_skip_known_answer(gpu):
    """Cin = 16 (two channels per child slot), Co = 8 (each repeated four times), worked by hand."""
    x = torch.arange(32, dtype=torch.float32).reshape(2, 16).to(torch.bfloat16)  # x[p, k] = 16p + k
    src = torch.tensor([3, 8 + 5, 8 * 9], dtype=torch.int32)  # (p=0, s=3), (p=1, s=5), outside x
    hg = torch.full((3, 8), 0.5, dtype=torch.bfloat16, device=gpu)
    sp.add_skip(hg, x.to(gpu), src.to(gpu))
    exp = [[6.5] * 4 + [7.5] * 4, [26.5] * 4 + [27.5] * 4, [0.5] * 8]
    assert hg.float().cpu().tolist() == exp
    with pytest.raises(RuntimeError):  # Co = 12: not a multiple of 8
        sp.add_skip(torch.zeros((3, 12), dtype=torch.bfloat16, device=gpu), x.to(gpu), src.to(gpu))


def test_upsample_block(gpu):
    """The reference's second half of an upsample block (src/sdec.cu:76-84) -- gather the conv1 output's child rows,
    LayerNorm, SiLU, conv2, skip add -- composed two ways from this library's entry points:
      (a) gather_ln_act(h1, src) then subm_conv_fused on the gathered rows, then add_skip;
      (b) ln_act of every parent sub-row (row-wise, so the same rows) then subm_conv_gathered(src), then add_skip;
    (a) and (b) are bit-identical, and both match the fp32 chain (oracle conv) to the conv's bf16 bar."""
    import oracle
    from spconv_amd import workloads as W
    par = W.shell_coords(W.CONFIGS["c1"])
    n, Cin, Co = len(par), 128, 64
    lg = W.keep_logits(n, 0.35, 5)
    ch, src = sp.subdivide(torch.from_numpy(par).to(gpu), torch.from_numpy(lg.view(np.int16)).to(gpu).view(torch.float16))
    m = len(ch)
    print(f"upsample block parents={n} children={m}", flush=True)
    g = torch.Generator().manual_seed(9)
    x = torch.randn((n, Cin), generator=g).to(torch.bfloat16)
    h1 = torch.randn((n, 8 * Co), generator=g).to(torch.bfloat16)  # conv1's output: 8 child slots of Co channels
    w, b = W.conv_params(W.Config("t", 0, 0, (0, 0), False, 0, Co, Co, "bf16", "", 21))
    wq = torch.from_numpy(w).to(torch.bfloat16)
    cache = sp.build_neighbors(ch.contiguous())
    xg, h1g, wg, bg = x.to(gpu), h1.to(gpu).view(8 * n, Co), wq.to(gpu), torch.from_numpy(b).to(gpu)

    ya = sp.subm_conv_fused(sp.gather_ln_act(h1g, src, 0), wg, bg, cache)
    sp.add_skip(ya, xg, src)
    yb = sp.subm_conv_gathered(sp.gather_ln_act(h1g), src, 0, wg, bg, cache)
    sp.add_skip(yb, xg, src)
    assert torch.equal(ya, yb)

    hc = h1.float().view(8 * n, Co)[src.cpu().long()]
    a = torch.nn.functional.silu(torch.nn.functional.layer_norm(hc, (Co,), eps=1e-6)).to(torch.bfloat16).float()
    nbr, _, _, _ = oracle.build_neighbors(ch.cpu().numpy())
    y32 = torch.from_numpy(oracle.conv(a.numpy(), wq.float().numpy(), b, nbr)).to(torch.bfloat16)
    ref = skip_reference(y32, x, src.cpu()).float().numpy()
    yr = ya.float().cpu().numpy()
    rel = np.linalg.norm(yr - ref) / np.linalg.norm(ref)
    err = np.abs(yr - ref)
    assert rel <= 3e-3 and np.all(err <= np.maximum(2e-2, 2 * ulp(ref, torch.bfloat16))), (rel, err.max())
    # (c) conv2 and the skip add in one pass (one rounding instead of two): same bar against the fp32 chain
    yc = sp.subm_conv_skip(sp.gather_ln_act(h1g, src, 0), wg, bg, cache, xg, src).float().cpu().numpy()
    ref32 = y32.float().numpy() + (skip_reference(torch.zeros_like(y32), x, src.cpu()).float().numpy())
    relc = np.linalg.norm(yc - ref32) / np.linalg.norm(ref32)
    errc = np.abs(yc - ref32)
    assert relc <= 3e-3 and np.all(errc <= np.maximum(2e-2, 2 * ulp(ref32, torch.bfloat16))), (relc, errc.max())


@pytest.mark.parametrize("Cin,Ci", [(64, 64), (128, 64), (256, 64), (512, 64), (128, 128)])
def test_conv_skip(gpu, Cin, Ci):
    """subm_conv_skip (rep = 8, 4, 2, 1 on the fused 64 -> 64 path; Ci = 128 runs conv then add_skip) against the
    fp32 oracle conv plus the skip in fp32, rounded once: the conv's bf16 bar."""
    import oracle
    from spconv_amd import workloads as W
    par = W.shell_coords(W.CONFIGS["c1"])
    n, Co = len(par), 64
    ch, src = sp.subdivide(torch.from_numpy(par).to(gpu),
                           torch.from_numpy(W.keep_logits(n, 0.4, 8).view(np.int16)).to(gpu).view(torch.float16))
    m = len(ch)
    print(f"conv_skip case Cin={Cin} Ci={Ci} children={m}", flush=True)
    g = torch.Generator().manual_seed(Cin + Ci)
    x = torch.randn((m, Ci), generator=g).to(torch.bfloat16)
    xs = torch.randn((n, Cin), generator=g).to(torch.bfloat16)
    w, b = W.conv_params(W.Config("t", 0, 0, (0, 0), False, 0, Ci, Co, "bf16", "", 41))
    wq = torch.from_numpy(w).to(torch.bfloat16)
    cache = sp.build_neighbors(ch.contiguous())
    for act in (0, 1):
        y = sp.subm_conv_skip(x.to(gpu), wq.to(gpu), torch.from_numpy(b).to(gpu), cache, xs.to(gpu), src, act=act)
        nbr, _, _, _ = oracle.build_neighbors(ch.cpu().numpy())
        conv = oracle.conv(x.float().numpy(), wq.float().numpy(), b, nbr, act=act)
        ref = conv + skip_reference(torch.zeros((m, Co), dtype=torch.bfloat16), xs, src.cpu()).float().numpy()
        yr = y.float().cpu().numpy()
        rel = np.linalg.norm(yr - ref) / np.linalg.norm(ref)
        err = np.abs(yr - ref)
        assert rel <= 3e-3 and np.all(err <= np.maximum(2e-2, ulp(ref, torch.bfloat16))), (act, rel, err.max())


@pytest.mark.parametrize("fused", ["1", "0"])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_conv_preln(gpu, monkeypatch, dt, fused):
    """subm_conv_preln (fused = 1: gather + LayerNorm + SiLU + conv + skip in the halo kernel; 0: the two-pass
    default) equals gather_ln_act followed by
    subm_conv_skip / subm_conv_fused bit for bit: with and without the skip, the affine terms and the SiLU, through
    the c2s map (shift 0, an upsample block's h1 sub-rows), through a shift-3 map, with no map, and with map entries
    outside the source (those rows are act(beta), as gather_ln_act makes them). The composition itself is checked
    against torch + the oracle in test_upsample_block."""
    from spconv_amd import workloads as W
    par = W.shell_coords(W.CONFIGS["c1"])
    n, Co = len(par), 64
    ch, src = sp.subdivide(torch.from_numpy(par).to(gpu),
                           torch.from_numpy(W.keep_logits(n, 0.35, 6).view(np.int16)).to(gpu).view(torch.float16))
    m = len(ch)
    monkeypatch.setenv("SPCONV_PRELN_FUSED", fused)
    print(f"preln case dt={dt} fused={fused} parents={n} children={m}", flush=True)
    g = torch.Generator().manual_seed(17)
    h1 = (torch.randn((8 * n, Co), generator=g) * 1.5 + 0.3).to(dt).to(gpu)  # h1 sub-rows, read through src
    hp = torch.randn((n, Co), generator=g).to(dt).to(gpu)  # parent rows, read through src >> 3
    hc = torch.randn((m, Co), generator=g).to(dt).to(gpu)  # child rows, no map
    xs = torch.randn((n, 128), generator=g).to(dt).to(gpu)
    w, b = W.conv_params(W.Config("t", 0, 0, (0, 0), False, 0, Co, Co, "bf16", "", 23))
    wg, bg = torch.from_numpy(w).to(dt).to(gpu), torch.from_numpy(b).to(gpu)
    gamma = (torch.rand(Co, generator=g) + 0.5).to(gpu)
    beta = (torch.randn(Co, generator=g) * 0.2).to(gpu)
    bad = src.clone()
    bad[::97] = 8 * n + 5  # outside the source rows
    cache = sp.build_neighbors(ch.contiguous())
    cases = [(h1, src, 0), (hp, src, 3), (hc, None, 0), (h1, bad, 0)]
    for k, (xsrc, rmap, shift) in enumerate(cases):
        for affine in (False, True):
            for pre_act in (0, 1):
                ga, be = (gamma, beta) if affine else (None, None)
                h = sp.gather_ln_act(xsrc, rmap, shift, ga, be, 1e-6, pre_act)
                ref = sp.subm_conv_skip(h, wg, bg, cache, xs, src, act=1)
                y = sp.subm_conv_preln(xsrc, wg, bg, cache, rmap, shift, ga, be, 1e-6, pre_act, act=1, x_skip=xs,
                                       skip_src=src)
                assert torch.equal(y, ref), (k, affine, pre_act, "skip")
                ref2 = sp.subm_conv_fused(h, wg, bg, cache, act=0)
                y2 = sp.subm_conv_preln(xsrc, wg, bg, cache, rmap, shift, ga, be, 1e-6, pre_act, act=0)
                assert torch.equal(y2, ref2), (k, affine, pre_act, "no skip")


def test_conv_preln_spill_and_ci128(gpu, monkeypatch):
    """subm_conv_preln with the one-kernel form requested, on a cache with spill tiles (it takes gather_ln_act + the
    conv) and at Ci = 128 on the opt-in 128-channel halo kernel and on the gathering kernel: bit for bit the
    composition."""
    from test_gpu_conv import mixed_spill_coords
    c = mixed_spill_coords()
    n = len(c)
    print(f"preln spill case rows={n}", flush=True)
    cache = sp.build_neighbors(torch.from_numpy(c).to(gpu))
    g = torch.Generator().manual_seed(5)
    monkeypatch.setenv("SPCONV_PRELN_FUSED", "1")
    for Ci in (64, 128):
        x = (torch.randn((n, Ci), generator=g) + 0.2).to(torch.bfloat16).to(gpu)
        w = (torch.randn((64, 27, Ci), generator=g) / (27 * Ci) ** 0.5).to(torch.bfloat16).to(gpu)
        b = (torch.randn(64, generator=g) * 0.1).to(gpu)
        gamma = (torch.rand(Ci, generator=g) + 0.5).to(gpu)
        beta = (torch.randn(Ci, generator=g) * 0.1).to(gpu)
        for mode in ("0", "1"):
            monkeypatch.setenv("SPCONV_HALO128", mode)
            ref = sp.subm_conv_fused(sp.gather_ln_act(x, None, 0, gamma, beta, 1e-5, 1), w, b, cache, act=1)
            y = sp.subm_conv_preln(x, w, b, cache, None, 0, gamma, beta, 1e-5, 1, act=1)
            assert torch.equal(y, ref), (Ci, mode)
