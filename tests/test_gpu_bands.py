"""GPU: frames rendered in screen bands (gaussian_splatting/rasterizer/bands.py).

Each band is rasterized through the unchanged surface from the frame's
projection with the means moved up by the band's first row, so each band is
held to the forward parity bar against the oracle on the same inputs, and the
stacked frame to a whole-frame render.  Config c5 at its full size (5M
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
from gaussian_splatting.rasterizer.bands import band_rows
from helpers import assert_bitwise, oracle_forward, scene_arrays
from oracle import oracle as orc
from test_gpu_parity import _np, gpu_forward

pytestmark = pytest.mark.gpu

NAMES = ("mu", "q", "s", "alpha", "A", "k_j")


def test_each_band_matches_the_oracle(crc, device):
    """c5's distributions at 30k Gaussians, 400x224, in 64-row bands (the last
    one 32 rows): each band's keys, ids, ranges, n_contrib, image and final T
    bit-exact against the oracle rasterizing the same moved means."""
    sc = synthetic.config_scene("c5", requires_grad=False, n=30_000, width=400, height=224)
    a = scene_arrays(sc)
    fw, want = gpu_forward(crc, a, device), oracle_forward(a)
    t, n = fw["tensors"], a["mu"].shape[0]
    depth = torch.from_numpy(fw["depth"]).to(device)
    for y0, h in band_rows(a["H"], 64):
        print(f"[gpu] band at row {y0}, {h} rows", flush=True)
        mb = t["mean2d"] - t["mean2d"].new_tensor([0.0, float(y0)])
        img, ids, rng, fT, nc, keys = crc.rasterize_with_keys(n, depth, mb, t["cov2d"], t["colors"],
                                                              t["alpha"], h, a["W"])
        mb_np = (want["mean2d"] - np.array([0.0, y0], np.float32)).astype(np.float32)
        wi, wids, wr, wfT, wnc, wkeys = orc.rasterize(want["depth"], mb_np, want["cov2d"],
                                                      want["colors"], a["alpha"], h, a["W"])
        assert_bitwise(_np(keys).view(np.uint64), wkeys, "sorted keys")
        assert_bitwise(_np(ids), wids, "sorted_ids")
        assert_bitwise(_np(rng), wr, "tile_ranges")
        assert_bitwise(_np(nc), wnc, "n_contrib")
        assert_bitwise(_np(img), wi, "img")
        assert_bitwise(_np(fT), wfT, "final_T")


def test_banded_glue_equals_the_whole_frame(device):
    """rasterize_bands against rasterize on a frame that fits: the image bit
    for bit, the parameter gradients and last_mean2d_grad within 1e-6
    relative (the same terms, summed per band first), the radii identical."""
    sc = synthetic.config_scene("c3", device=device, n=20_000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    w = torch.linspace(0.5, 1.5, 480 * 272 * 3, device=device).view(272, 480, 3)

    def run(render):
        for nm in NAMES:
            getattr(g, nm).grad = None
        img = render()
        (img * w).sum().backward()
        return (img.detach().clone(), [getattr(g, nm).grad.clone() for nm in NAMES],
                RasterizeFunction.last_mean2d_grad.clone(), RasterizeFunction.last_radii2d.clone())

    bi, bg, bm, br = run(lambda: rasterize_bands(g, view, 96))
    wi, wg, wm, wr = run(lambda: rasterize(g, view))
    assert_bitwise(_np(bi), _np(wi), "image")
    assert_bitwise(_np(br), _np(wr), "radii")
    for got, want, nm in zip(bg + [bm], wg + [wm], NAMES + ("last_mean2d_grad",)):
        err = (got - want).norm() / want.norm().clamp_min(1e-30)
        assert err <= 1e-6, f"d {nm}: {err:.2e}"


def test_bands_without_gaussians(device):
    """Every Gaussian above row 130 of a 272-row frame: of the 64-row bands,
    the last two hold no pair at all (empty lists through rasterize and its
    backward).  The stacked image is the whole frame's bit for bit, those
    bands are zero, and the gradients match rasterize's within 1e-6."""
    sc = synthetic.config_scene("c3", device=device, n=2000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    with torch.no_grad():
        g.mu[:, 1] = -0.5 - 0.5 * g.mu[:, 1].abs()  # y in [-1, -0.5]: projected near the top
    w = torch.linspace(0.5, 1.5, 480 * 272 * 3, device=device).view(272, 480, 3)

    def run(render):
        for nm in NAMES:
            getattr(g, nm).grad = None
        img = render()
        (img * w).sum().backward()
        return img.detach().clone(), [getattr(g, nm).grad.clone() for nm in NAMES]

    bi, bg = run(lambda: rasterize_bands(g, view, 64))
    wi, wg = run(lambda: rasterize(g, view))
    assert_bitwise(_np(bi), _np(wi), "image")
    assert float(bi[192:].abs().max()) == 0.0 and float(bi[:64].abs().max()) > 0.0
    for got, want, nm in zip(bg, wg, NAMES):
        err = (got - want).norm() / want.norm().clamp_min(1e-30)
        assert err <= 1e-6, f"d {nm}: {err:.2e}"


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
        m2, c2, d = crc.project(n, g.mu, g.q, g.s, view["R"], view["T"], view["fx"], view["fy"],
                                view["cx"], view["cy"])
        col = crc.SH(n, (-(view["R"].T @ view["T"])).contiguous(), g.mu, g.A, g.k_j)
        op = torch.sigmoid(g.alpha)
        for y0, h in band_rows(view["height"], 256):
            mb = m2 - m2.new_tensor([0.0, float(y0)])
            out = crc.rasterize(n, d, mb, c2, col, op, h, view["width"])
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
