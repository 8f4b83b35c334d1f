"""GPU parity of the one-pass ConvNeXt tail (LayerNorm + affine -> Linear 4C + SiLU -> Linear C -> + x) against
torch fp32 on the same inputs.

Two references:
  * `emulated`: torch fp32 with the kernel's two roundings to the operand dtype (the normalized rows before the
    first product, the SiLU output before the second); the kernel differs only in accumulation order and in SiLU's
    fast exp/reciprocal, so it must agree to rel-L2 <= 2e-3 and max-abs <= 3e-2 (bf16 output rounding alone is
    ~1.7e-3 relative);
  * `fp32`: no intermediate rounding; rel-L2 <= 1e-2 (the intermediate bf16 roundings, propagated).
"""
import numpy as np
import pytest
import torch

import spconv_amd as sp

pytestmark = pytest.mark.gpu


def make(N, C, dt, pdt, seed):
    g = torch.Generator().manual_seed(seed)
    h = (torch.randn((N, C), generator=g) * 3 + 1).to(dt)
    x = torch.randn((N, C), generator=g).to(dt)
    gamma = (torch.rand(C, generator=g) + 0.5).to(pdt)
    beta = (torch.randn(C, generator=g) * 0.2).to(pdt)
    w1 = (torch.randn((4 * C, C), generator=g) / C ** 0.5).to(dt)
    b1 = (torch.randn(4 * C, generator=g) * 0.1).to(pdt)
    w2 = (torch.randn((C, 4 * C), generator=g) / (4 * C) ** 0.5).to(dt)
    b2 = (torch.randn(C, generator=g) * 0.1).to(pdt)
    return h, x, gamma, beta, w1, b1, w2, b2


def reference(h, x, gamma, beta, w1, b1, w2, b2, eps, dt=None):
    r = (lambda t: t.to(dt).float()) if dt is not None else (lambda t: t)
    f = lambda t: None if t is None else t.float()
    a = r(torch.nn.functional.layer_norm(h.float(), (h.shape[1],), f(gamma), f(beta), eps))
    a = r(torch.nn.functional.silu(a @ w1.float().T + (0 if b1 is None else b1.float())))
    return a @ w2.float().T + (0 if b2 is None else b2.float()) + x.float()


def rel(a, b):
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


def check(y, args, eps, dt, what):
    y = y.float().cpu()
    em = reference(*args, eps, dt)
    f32 = reference(*args, eps)
    r_em, mx, r_32 = rel(y, em), float((y - em).abs().max()), rel(y, f32)
    print(f"{what}: rel-L2 {r_em:.2e} max-abs {mx:.2e} vs emulated, rel-L2 {r_32:.2e} vs fp32", flush=True)
    assert torch.isfinite(y).all(), what
    assert r_em <= 2e-3 and mx <= 3e-2 and r_32 <= 1e-2, what


@pytest.mark.parametrize("C", [64, 128, 256, 512, 1024])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_convnext_mlp(gpu, C, dt):
    print(f"mlp case C={C} dt={dt}", flush=True)
    for N, pdt in ((3001, torch.float32), (5, dt)):
        args = make(N, C, dt, pdt, C + N)
        y = sp.convnext_mlp(*[a.to(gpu) for a in args], eps=1e-6)
        check(y, args, 1e-6, dt, f"C={C} N={N} {dt} params {pdt}")


@pytest.mark.parametrize("C", [64, 128, 512])
def test_convnext_mlp_many_tiles_in_place(gpu, C):
    """More row tiles than workgroups (the persistent loop and, for C = 128, the weight stream across tiles; for
    C = 512 the three-pass form), no affine and no biases, output written over h."""
    N = {64: 70001, 128: 140001, 512: 20001}[C]
    print(f"mlp many-tiles case C={C} N={N}", flush=True)
    h, x, _, _, w1, _, w2, _ = make(N, C, torch.bfloat16, torch.float32, 5)
    hg = h.to(gpu)
    y = sp.convnext_mlp(hg, x.to(gpu), None, None, w1.to(gpu), None, w2.to(gpu), None, eps=1e-5, out=hg)
    assert y.data_ptr() == hg.data_ptr()
    check(hg, (h, x, None, None, w1, None, w2, None), 1e-5, torch.bfloat16, f"C={C} N={N} in place")


def test_convnext_mlp_errors(gpu):
    h = torch.zeros((10, 96), dtype=torch.bfloat16, device=gpu)
    w1 = torch.zeros((384, 96), dtype=torch.bfloat16, device=gpu)
    w2 = torch.zeros((96, 384), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError):  # C = 96 unsupported
        sp.convnext_mlp(h, h, None, None, w1, None, w2, None)
    e = torch.zeros((0, 64), dtype=torch.bfloat16, device=gpu)
    w1 = torch.zeros((256, 64), dtype=torch.bfloat16, device=gpu)
    w2 = torch.zeros((64, 256), dtype=torch.bfloat16, device=gpu)
    assert sp.convnext_mlp(e, e, None, None, w1, None, w2, None).shape == (0, 64)
    h = torch.zeros((10, 384), dtype=torch.bfloat16, device=gpu)  # C = 384: neither form
    w1 = torch.zeros((1536, 384), dtype=torch.bfloat16, device=gpu)
    w2 = torch.zeros((384, 1536), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="512, 1024"):
        sp.convnext_mlp(h, h, None, None, w1, None, w2, None)
