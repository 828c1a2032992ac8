"""The reference's finite-difference checks (tests/test_cuda_backward.py:53-263) on the
HIP build: same scenes, same torch.autograd.gradcheck tolerances (fp32, eps 1e-3,
atol 1e-3, rtol 1e-2, nondet_tol 1e-4), each wrapping the raw custom_rasterizer_cuda
calls or RasterizeFunction end to end."""

from __future__ import annotations

import pytest
import torch
from torch.autograd import gradcheck

from gaussian_splatting.rasterizer.rasterize import RasterizeFunction

pytestmark = pytest.mark.gpu

GRADCHECK = dict(eps=1e-3, atol=1e-3, rtol=1e-2, nondet_tol=1e-4, check_batched_grad=False,
                 raise_exception=True)


def _leaf(x):
    return x.detach().contiguous().clone().requires_grad_(True)


def test_projection_backward_matches_finite_differences(crc, device):
    rotation = torch.eye(3, device=device)
    translation = torch.zeros(3, device=device)
    fx = fy = 200.0
    cx = cy = 100.0
    mu = _leaf(torch.tensor([[0.30, -0.20, 3.5], [-0.25, 0.15, 5.0]], device=device))
    quat = torch.tensor([1.0, 0.15, -0.05, 0.02], device=device)
    q = _leaf((quat / quat.norm()).expand(2, 4).clone())
    s = _leaf(torch.tensor([[-2.2, -2.0, -1.8], [-2.5, -2.1, -2.3]], device=device))

    class Project(torch.autograd.Function):
        @staticmethod
        def forward(ctx, means, quats, scales):
            m2, c2, _ = crc.project(means.shape[0], means.contiguous(), quats.contiguous(),
                                    scales.contiguous(), rotation, translation, fx, fy, cx, cy)
            ctx.save_for_backward(means, quats, scales)
            return m2, c2

        @staticmethod
        def backward(ctx, gm, gc):
            means, quats, scales = ctx.saved_tensors
            return crc.backwards_projection(gm.contiguous(), gc.contiguous(), means, quats, scales,
                                            rotation, translation, fx, fy, cx, cy)

    m2, c2 = Project.apply(mu, q, s)
    assert torch.isfinite(m2).all() and torch.isfinite(c2).all()
    assert float(m2.detach().abs().sum()) > 1.0 and float(c2.detach().abs().sum()) > 0.1
    # fp32 central differences at eps 1e-3 of outputs near 43 px^2 carry ~ulp(43)/eps
    # ~ 2e-3 of rounding noise, above atol; the numerical Jacobian is therefore taken
    # from the float64 forward (the CPU oracle, whose fp32 forward the GPU matches bit
    # for bit) at the same fp32 inputs, and the GPU's analytical Jacobian is held to
    # the reference's tolerances against it.
    import numpy as np
    from oracle import oracle as orc

    inputs = {"mu": mu, "q": q, "s": s}
    n_out = 10
    for name, x in inputs.items():
        ana = np.zeros((n_out, x.numel()))
        for o in range(n_out):
            gm = torch.zeros(2, 2, device=device)
            gc = torch.zeros(2, 3, device=device)
            (gm if o < 4 else gc).view(-1)[o if o < 4 else o - 4] = 1.0
            grads = crc.backwards_projection(gm, gc, mu.detach(), q.detach(), s.detach(),
                                             rotation, translation, fx, fy, cx, cy)
            ana[o] = grads[list(inputs).index(name)].detach().cpu().numpy().reshape(-1)
        num = np.zeros_like(ana)
        base = {k: v.detach().cpu().numpy().astype(np.float64) for k, v in inputs.items()}
        for j in range(x.numel()):
            outs = []
            for sgn in (1, -1):
                p = {k: v.copy() for k, v in base.items()}
                p[name].reshape(-1)[j] += sgn * GRADCHECK["eps"]
                a2, b2, _ = orc.project(p["mu"], p["q"], p["s"], np.eye(3), np.zeros(3), fx, fy, cx,
                                        cy, dtype=np.float64)
                outs.append(np.concatenate([a2.reshape(-1), b2.reshape(-1)]))
            num[:, j] = (outs[0] - outs[1]) / (2 * GRADCHECK["eps"])
        bad = np.abs(ana - num) > GRADCHECK["atol"] + GRADCHECK["rtol"] * np.abs(num)
        assert not bad.any(), (name, np.argwhere(bad)[:4], ana[bad][:4], num[bad][:4])


def test_sh_backward_matches_finite_differences(crc, device):
    camera = torch.zeros(3, device=device)
    mu = _leaf(torch.tensor([[0.40, -0.30, 2.5], [-0.20, 0.50, 3.0]], device=device))
    albedo = _leaf(torch.zeros(2, 3, device=device))
    k_j = _leaf(torch.linspace(-0.005, 0.005, 90, device=device).reshape(2, 15, 3))

    class SH(torch.autograd.Function):
        @staticmethod
        def forward(ctx, means, alb, coeff):
            ctx.save_for_backward(means, alb, coeff)
            return crc.SH(means.shape[0], camera, means.contiguous(), alb.contiguous(),
                          coeff.contiguous())

        @staticmethod
        def backward(ctx, gcol):
            means, alb, coeff = ctx.saved_tensors
            dA, dk, dmu = crc.backwards_SH(gcol.contiguous(), means, alb, coeff, camera)
            return dmu, dA, dk

    col = SH.apply(mu, albedo, k_j)
    assert float(col.detach().min()) > 0.05 and float(col.detach().max()) < 0.95
    assert gradcheck(SH.apply, (mu, albedo, k_j), **GRADCHECK)


def test_rasterize_backward_matches_finite_differences(crc, device):
    H = W = 16
    mean_2d = _leaf(torch.tensor([[8.0, 8.0]], device=device))
    cov_2d = _leaf(torch.tensor([[4.0, 0.0, 4.0]], device=device))
    colors = _leaf(torch.tensor([[0.25, 0.45, 0.70]], device=device))
    alpha = _leaf(torch.tensor([[0.6]], device=device))
    depths = torch.tensor([2.0], device=device)

    class Raster(torch.autograd.Function):
        @staticmethod
        def forward(ctx, means, cov, rgb, opacity):
            img, ids, ranges, fT, nc = crc.rasterize(means.shape[0], depths, means.contiguous(),
                                                     cov.contiguous(), rgb.contiguous(),
                                                     opacity.contiguous(), H, W)
            ctx.save_for_backward(means, cov, rgb, opacity, ids, ranges, fT, nc)
            return img

        @staticmethod
        def backward(ctx, g):
            means, cov, rgb, opacity, ids, ranges, fT, nc = ctx.saved_tensors
            return crc.backwards_rasterization(g.contiguous(), means, cov, rgb, opacity, ids,
                                               ranges, fT, nc, means.shape[0], H, W)

    def center(*args):
        return Raster.apply(*args)[6:10, 6:10].sum()

    assert float(center(mean_2d, cov_2d, colors, alpha).detach()) > 1e-2
    assert gradcheck(center, (mean_2d, cov_2d, colors, alpha), **GRADCHECK)


def test_full_pipeline_backward_matches_finite_differences(crc, device):
    H = W = 16
    rotation = torch.eye(3, device=device)
    translation = torch.zeros(3, device=device)
    mu = _leaf(torch.tensor([[0.05, -0.04, 4.0]], device=device))
    quat = torch.tensor([1.0, 0.1, -0.05, 0.02], device=device)
    q = _leaf((quat / quat.norm()).reshape(1, 4))
    s = _leaf(torch.full((1, 3), -2.0, device=device))
    alpha = _leaf(torch.tensor([[0.5]], device=device))
    albedo = _leaf(torch.zeros(1, 3, device=device))
    k_j = _leaf(torch.linspace(-0.005, 0.005, 45, device=device).reshape(1, 15, 3))

    def pipeline(m, qq, ss, op, alb, coeff):
        img = RasterizeFunction.apply(m, qq, ss, op, alb, coeff, rotation, translation, 16.0, 16.0,
                                      8.0, 8.0, H, W)
        return img[7:9, 7:9].sum()

    assert float(pipeline(mu, q, s, alpha, albedo, k_j).detach()) > 1e-3
    assert gradcheck(pipeline, (mu, q, s, alpha, albedo, k_j), **GRADCHECK)
