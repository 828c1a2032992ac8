"""Pins of the loss oracle (oracle/loss_oracle.py), CPU only: the window's closed
form, SSIM's identities (SSIM(x, x) = 1, symmetry, the constant-image closed
form), a brute-force per-window evaluation with 2D weights, torchmetrics'
padded-then-cropped pipeline restated with torch (float64), and the gradient
against torch autograd of an independent torch restatement and against
central finite differences."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import loss_oracle as lo


def _imgs(seed=0, H=24, W=29, lo_=0.05, hi=0.95):
    rng = np.random.default_rng(seed)
    a = rng.uniform(lo_, hi, (H, W, 3))
    b = np.clip(a + rng.normal(0, 0.15, (H, W, 3)), lo_, hi)
    return a, b


def test_window_closed_form():
    w = lo.gaussian_window()
    assert w.size == 11 and abs(w.sum() - 1.0) < 1e-15
    assert np.allclose(w, w[::-1], rtol=0, atol=0)
    # neighbouring taps: ratio exp((2k + 1) / (2 sigma^2)) for d = k -> k + 1
    for k in range(5):
        assert np.isclose(w[5 + k] / w[6 + k], np.exp((2 * k + 1) / (2 * 1.5 ** 2)), rtol=1e-14)


def test_ssim_identities():
    a, b = _imgs(1)
    assert abs(lo.ssim(a, a) - 1.0) < 1e-12
    assert abs(lo.ssim(a, b) - lo.ssim(b, a)) < 1e-15
    s = lo.ssim_map(a, b)
    assert s.shape == (a.shape[0] - 10, a.shape[1] - 10, 3)
    assert np.all(s <= 1.0 + 1e-12) and np.all(s >= -1.0 - 1e-12)


@pytest.mark.parametrize("ca,cb", [(0.3, 0.3), (0.2, 0.7), (0.0, 1.0), (1.0, 0.9)])
def test_constant_images_closed_form(ca, cb):
    a = np.full((13, 17, 3), ca)
    b = np.full((13, 17, 3), cb)
    want = (2 * ca * cb + lo.C1) / (ca * ca + cb * cb + lo.C1)
    assert abs(lo.ssim(a, b) - want) < 1e-12


def test_brute_force_windows():
    a, b = _imgs(2, H=15, W=14)
    w1 = lo.gaussian_window()
    w2 = np.outer(w1, w1)
    H, W = a.shape[:2]
    want = np.zeros((H - 10, W - 10, 3))
    for i in range(H - 10):
        for j in range(W - 10):
            for c in range(3):
                x = a[i:i + 11, j:j + 11, c]
                y = b[i:i + 11, j:j + 11, c]
                mx, my = (w2 * x).sum(), (w2 * y).sum()
                vx = (w2 * x * x).sum() - mx * mx
                vy = (w2 * y * y).sum() - my * my
                cxy = (w2 * x * y).sum() - mx * my
                want[i, j, c] = ((2 * mx * my + lo.C1) * (2 * cxy + lo.C2)) / (
                    (mx * mx + my * my + lo.C1) * (vx + vy + lo.C2))
    assert np.abs(lo.ssim_map(a, b) - want).max() < 1e-13


def _torch_ssim_padded(a, b):
    """torchmetrics' pipeline as its source reads: reflect padding by the
    window radius, grouped conv with the 2D Gaussian, the index map, then the
    crop of the radius, mean."""
    x = torch.from_numpy(a).permute(2, 0, 1).unsqueeze(0)
    y = torch.from_numpy(b).permute(2, 0, 1).unsqueeze(0)
    w1 = torch.from_numpy(lo.gaussian_window())
    k = torch.outer(w1, w1).expand(3, 1, 11, 11).contiguous()
    p = 5
    xp = torch.nn.functional.pad(x, (p, p, p, p), mode="reflect")
    yp = torch.nn.functional.pad(y, (p, p, p, p), mode="reflect")
    inp = torch.cat((xp, yp, xp * xp, yp * yp, xp * yp))
    out = torch.nn.functional.conv2d(inp, k, groups=3)
    mx, my, exx, eyy, exy = out.split(1)
    # the variances clamped at 0, as torchmetrics after 1.0
    sxx, syy, sxy = (exx - mx * mx).clamp(min=0.0), (eyy - my * my).clamp(min=0.0), exy - mx * my
    s = ((2 * mx * my + lo.C1) * (2 * sxy + lo.C2)) / ((mx * mx + my * my + lo.C1) * (sxx + syy + lo.C2))
    return s[..., p:-p, p:-p].mean()


def test_padded_then_cropped_equals_valid():
    a, b = _imgs(3, H=33, W=40)
    assert abs(float(_torch_ssim_padded(a, b)) - lo.ssim(a, b)) < 1e-13


def _torch_loss(r, g, lam):
    rc, gc = r.clamp(0.0, 1.0), g.clamp(0.0, 1.0)
    l1 = torch.mean(torch.abs(g - r))
    x, y = rc.permute(2, 0, 1).unsqueeze(0), gc.permute(2, 0, 1).unsqueeze(0)
    w1 = torch.from_numpy(lo.gaussian_window())
    k = torch.outer(w1, w1).expand(3, 1, 11, 11).contiguous()
    conv = lambda t: torch.nn.functional.conv2d(t, k, groups=3)
    mx, my = conv(x), conv(y)
    sxx = (conv(x * x) - mx * mx).clamp(min=0.0)
    syy = (conv(y * y) - my * my).clamp(min=0.0)
    sxy = conv(x * y) - mx * my
    s = ((2 * mx * my + lo.C1) * (2 * sxy + lo.C2)) / ((mx * mx + my * my + lo.C1) * (sxx + syy + lo.C2))
    return (1 - lam) * l1 + lam * (1 - s.mean())


@pytest.mark.parametrize("lam", [0.2, 0.0, 1.0])
def test_gradient_matches_autograd(lam):
    rng = np.random.default_rng(4)
    r = rng.normal(0.5, 0.35, (21, 26, 3))  # some values outside [0, 1]
    g = rng.uniform(0, 1, (21, 26, 3))
    rt = torch.from_numpy(r).requires_grad_(True)
    loss = _torch_loss(rt, torch.from_numpy(g), lam)
    loss.backward()
    want = rt.grad.numpy()
    got = lo.l1_dssim_grad(r, g, lam, grad_loss=1.0)
    assert np.abs(got - want).max() <= 1e-12 * max(np.abs(want).max(), 1e-30) + 1e-18
    assert abs(lo.l1_dssim(r, g, lam)[0] - float(loss.detach())) < 1e-13


def test_gradient_finite_differences():
    r, g = _imgs(5, H=16, W=18, lo_=0.1, hi=0.9)
    grad = lo.l1_dssim_grad(r, g, 0.2, grad_loss=1.7)
    rng = np.random.default_rng(6)
    eps = 1e-6
    for _ in range(40):
        i, j, c = rng.integers(16), rng.integers(18), rng.integers(3)
        rp, rm = r.copy(), r.copy()
        rp[i, j, c] += eps
        rm[i, j, c] -= eps
        fd = 1.7 * (lo.l1_dssim(rp, g)[0] - lo.l1_dssim(rm, g)[0]) / (2 * eps)
        assert abs(fd - grad[i, j, c]) <= 1e-6 * max(abs(grad[i, j, c]), 1e-4)


def test_clamped_pixels_get_only_the_l1_term():
    r, g = _imgs(7, H=14, W=14)
    r[3, 4, 1] = 1.3
    r[8, 2, 0] = -0.2
    grad = lo.l1_dssim_grad(r, g, 0.2)
    n = r.size
    assert grad[3, 4, 1] == pytest.approx(0.8 / n)   # rendered above gt: +1/n of the L1 term
    assert grad[8, 2, 0] == pytest.approx(-0.8 / n)  # below gt


def test_index_derivatives_through_the_variance_clamp():
    """dS/d(mu_x, E[x^2], E[xy]) against torch autograd of the clamped index,
    on moments whose sigma_x^2 or sigma_y^2 lies below, at and above 0 (the
    clamp passes the gradient at 0, as torch's clamp backward)."""
    rng = np.random.default_rng(8)
    mx = rng.uniform(0.05, 0.95, 64)
    my = rng.uniform(0.05, 0.95, 64)
    vx = np.concatenate([rng.uniform(-2e-3, -1e-6, 16), np.zeros(16), rng.uniform(1e-6, 2e-2, 32)])
    vy = rng.permutation(np.concatenate([rng.uniform(-2e-3, -1e-6, 20), rng.uniform(1e-6, 2e-2, 44)]))
    exx, eyy = vx + mx * mx, vy + my * my
    exy = mx * my + rng.uniform(-5e-3, 5e-3, 64)
    t = [torch.from_numpy(a.copy()).requires_grad_(True) for a in (mx, my, exx, eyy, exy)]
    tmx, tmy, texx, teyy, texy = t
    sxx = (texx - tmx * tmx).clamp(min=0.0)
    syy = (teyy - tmy * tmy).clamp(min=0.0)
    sxy = texy - tmx * tmy
    st = ((2 * tmx * tmy + lo.C1) * (2 * sxy + lo.C2)) / (
        (tmx * tmx + tmy * tmy + lo.C1) * (sxx + syy + lo.C2))
    st.sum().backward()
    s, g1, g2, g3 = lo.index_derivatives(mx, my, exx, eyy, exy)
    assert np.allclose(s, st.detach().numpy(), rtol=1e-13, atol=0)
    for got, want in ((g1, tmx.grad), (g2, texx.grad), (g3, texy.grad)):
        want = want.numpy()
        assert np.allclose(got, want, rtol=1e-11, atol=1e-11 * np.abs(want).max())
    # below 0 the E[x^2] path carries nothing; above it, -S / B2
    assert np.all(g2[:16] == 0.0) and np.all(g2[16:] != 0.0)
