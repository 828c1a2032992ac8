"""GPU: frames rendered in screen bands (gaussian_splatting/rasterizer/bands.py).

Each band is a frame of its own through the unchanged surface, so each is held
to the forward parity bar against the oracle on the band's camera.  The glue
stacks the bands and sums their gradients.  Config c5 at its full size (5M
Gaussians at 3840x2160, ~1.1e10 pairs) is beyond the int32 pair lists of the
reference's surface (rasterize.cu:382-390): the whole frame is refused with an
error, and the banded frame is checked by size-independent properties.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splatting import synthetic
from gaussian_splatting.rasterizer import RasterizeFunction, rasterize, rasterize_bands
from gaussian_splatting.rasterizer.bands import band_views
from helpers import assert_bitwise, oracle_forward, scene_arrays
from test_gpu_parity import _check_forward, _np, gpu_forward

pytestmark = pytest.mark.gpu

NAMES = ("mu", "q", "s", "alpha", "A", "k_j")


def test_each_band_matches_the_oracle(crc, device):
    """c5's distributions at 30k Gaussians, 400x224, in 64-row bands (the last
    one 32 rows): every band bit-exact against the oracle on its camera."""
    sc = synthetic.config_scene("c5", requires_grad=False, n=30_000, width=400, height=224)
    a = scene_arrays(sc)
    for y0, v in band_views(sc.view, 64):
        print(f"[gpu] band at row {y0}, {v['height']} rows", flush=True)
        b = dict(a, cy=float(v["cy"]), H=int(v["height"]))
        _check_forward(gpu_forward(crc, b, device), oracle_forward(b))


def test_banded_glue_stacks_bands_and_sums_their_gradients(device):
    """rasterize_bands: the image is the bands' images stacked (bit for bit
    rasterize on each band's view); the parameter gradients are the sums of
    the bands' gradients (fp32 sums in another order: 1e-6 relative), and
    last_mean2d_grad is the sum of the bands' dL/d mean2d."""
    sc = synthetic.config_scene("c3", device=device, n=20_000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    w = torch.linspace(0.5, 1.5, 480 * 272 * 3, device=device).view(272, 480, 3)

    def clear():
        for nm in NAMES:
            getattr(g, nm).grad = None

    clear()
    img = rasterize_bands(g, view, 96)
    (img * w).sum().backward()
    banded = [getattr(g, nm).grad.clone() for nm in NAMES]
    banded_m2 = RasterizeFunction.last_mean2d_grad.clone()

    sums = [torch.zeros_like(x) for x in banded]
    m2_sum = None
    for y0, v in band_views(view, 96):
        clear()
        part = rasterize(g, v)
        assert_bitwise(_np(img[y0:y0 + v["height"]]), _np(part), f"band at row {y0}")
        (part * w[y0:y0 + v["height"]]).sum().backward()
        for acc, nm in zip(sums, NAMES):
            acc += getattr(g, nm).grad
        m = RasterizeFunction.last_mean2d_grad
        m2_sum = m.clone() if m2_sum is None else m2_sum + m
    for got, want, nm in zip(banded, sums, NAMES):
        err = (got - want).norm() / want.norm().clamp_min(1e-30)
        assert err <= 1e-6, f"d {nm}: {err:.2e}"
    err = (banded_m2 - m2_sum).norm() / m2_sum.norm()
    assert err <= 1e-6, f"last_mean2d_grad: {err:.2e}"


def test_c5_full_size_in_screen_bands(crc, device):
    """Config c5 at full size.  The whole frame needs more pairs than int32
    lists hold and is refused; in 256-row bands every band fits, the pairs add
    up to more than 2^31, the image is finite and in [0, 1], and the
    gradients are finite and deterministic."""
    print("[gpu] c5 full size: 5M Gaussians, 3840x2160", flush=True)
    sc = synthetic.config_scene("c5", device=device)
    g, view = sc.gaussians, sc.view
    with pytest.raises(RuntimeError, match="screen bands"):
        rasterize(g, view)
    pairs = []
    with torch.no_grad():
        n = g.mu.shape[0]
        for _, v in band_views(view, 256):
            m2, c2, d = crc.project(n, g.mu, g.q, g.s, v["R"], v["T"], v["fx"], v["fy"],
                                    v["cx"], v["cy"])
            col = crc.SH(n, (-(v["R"].T @ v["T"])).contiguous(), g.mu, g.A, g.k_j)
            out = crc.rasterize(n, d, m2, c2, col, torch.sigmoid(g.alpha), v["height"],
                                v["width"])
            pairs.append(out[1].numel())
            del out
    print(f"[gpu] c5 pairs per band: {pairs}", flush=True)
    assert sum(pairs) > 2**31 and max(pairs) < 2**31 - 65535

    def frame():
        for nm in NAMES:
            getattr(g, nm).grad = None
        img = rasterize_bands(g, view, 256)
        img.sum().backward()
        torch.cuda.synchronize()
        return img.detach(), [getattr(g, nm).grad.clone() for nm in NAMES]

    img, g1 = frame()
    assert img.shape == (2160, 3840, 3)
    assert torch.isfinite(img).all() and img.min() >= 0 and img.max() <= 1
    assert img.max() > 0
    for x, nm in zip(g1, NAMES):
        assert torch.isfinite(x).all(), nm
    print("[gpu] c5 second frame (determinism)", flush=True)
    img2, g2 = frame()
    assert torch.equal(img, img2)
    for x, y, nm in zip(g1, g2, NAMES):
        assert torch.equal(x, y), nm
    del img, img2, g1, g2
    torch.cuda.empty_cache()
