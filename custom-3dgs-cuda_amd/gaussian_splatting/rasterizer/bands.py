"""Screen-band rendering: frames whose (Gaussian, tile) pair count is beyond the
int32 lists of the rasterize surface (the reference keeps the pair count, the
offsets and ``sorted_ids`` in int, rasterize.cu:382-390, rasterize.h:7-8).

One autograd Function renders the frame as bands of whole tile rows:
- forward: the fused head (camera position, project, radii, SH, sigmoid) runs
  once; each band of rows [y0, y0 + h) is rasterized through the unchanged
  surface from the frame's projection with the means moved up by y0 rows;
- backward: each band's rasterize backward reads its rows of dL/dimage in
  place; their d mean2d, d cov2d, d colour and d opacity are summed, and the
  fused tail (SH and projection backward, the sigmoid's backward) runs once.

Band heights are multiples of the 16-pixel tile, so a band's tiles are the
frame's tiles.  Moving a mean by a whole number of rows is exact in fp32
whenever the mean lies at or below the band's top row, and then the band's
pixel offsets are the frame's bit for bit: the banded image equals a
whole-frame render.  Only a mean far above the band can round (its own last
bit), which can move that Gaussian's footprint in the band by that bit.
"""

from __future__ import annotations

import torch as t

import gaussian_splatting.rasterizer.rasterize as glue
from gaussian_splatting.rasterizer.rasterize import RasterizeFunction
from gaussian_splatting.scene.gaussian import gaussian

TILE = 16


def band_rows(height: int, band_height: int) -> list[tuple[int, int]]:
    """(y0, h) of each band, top to bottom."""
    if band_height <= 0 or band_height % TILE:
        raise ValueError(f"band_height must be a positive multiple of {TILE}, got {band_height}")
    return [(y0, min(band_height, height - y0)) for y0 in range(0, height, band_height)]


def band_views(view: dict, band_height: int) -> list[tuple[int, dict]]:
    """(y0, view of rows [y0, y0 + h)) for each band: the frame's camera with
    the principal point moved up by y0 (cy - y0) and height h.  A band rendered
    from this view through rasterize() is the band of the frame up to the
    rounding of cy - y0 inside the projection; rasterize_bands shifts the
    projected means instead, which is exact."""
    out = []
    for y0, h in band_rows(int(view["height"]), band_height):
        v = dict(view)
        v["cy"] = float(view["cy"]) - y0
        v["height"] = h
        out.append((y0, v))
    return out


class _RasterizeBandsFunction(t.autograd.Function):
    @staticmethod
    def forward(ctx, mu, q, s, alpha_logits, albedo, k_j, cam_rotation, cam_translation, fx, fy,
                cx, cy, height, width, band_height):
        crc = glue.crc
        if crc is None:
            raise ImportError("custom_rasterizer_cuda is not built. "
                              "Build it with: python custom-3dgs-cuda_amd/build.py")
        n = mu.shape[0]
        mu, q, s = mu.contiguous(), q.contiguous(), s.contiguous()
        alpha_logits, albedo, k_j = alpha_logits.contiguous(), albedo.contiguous(), k_j.contiguous()
        cam_rotation, cam_translation = cam_rotation.contiguous(), cam_translation.contiguous()
        fx, fy, cx, cy = float(fx), float(fy), float(cx), float(cy)
        H, W = int(height), int(width)
        mean_2d, cov_2d, depths, radii, colors, cam_position, opacity = crc.project_sh(
            n, mu, q, s, cam_rotation, cam_translation, fx, fy, cx, cy, albedo, k_j, alpha_logits)
        RasterizeFunction.last_radii2d = radii
        images, saved, rows = [], [], band_rows(H, band_height)
        for y0, h in rows:
            mean_b = mean_2d - mean_2d.new_tensor([0.0, float(y0)])
            img, ids, ranges, final_T, n_contrib = crc.rasterize(n, depths, mean_b, cov_2d, colors,
                                                                 opacity, h, W)
            images.append(img)
            saved += [mean_b, ids, ranges, final_T, n_contrib]
        ctx.save_for_backward(cov_2d, colors, opacity, mu, q, s, albedo, k_j, cam_rotation,
                              cam_translation, cam_position, *saved)
        ctx.rows, ctx.n, ctx.W, ctx.fx, ctx.fy = rows, n, W, fx, fy
        return t.cat(images, dim=0)

    @staticmethod
    def backward(ctx, grad_output):
        crc = glue.crc
        (cov_2d, colors, opacity, mu, q, s, albedo, k_j, cam_rotation, cam_translation,
         cam_position, *saved) = ctx.saved_tensors
        n, W = ctx.n, ctx.W
        sums = None
        for i, (y0, h) in enumerate(ctx.rows):
            mean_b, ids, ranges, final_T, n_contrib = saved[5 * i:5 * i + 5]
            part = crc.backwards_rasterization_strided(
                grad_output[y0:y0 + h], mean_b, cov_2d, colors, opacity, ids, ranges, final_T,
                n_contrib, n, h, W)
            sums = list(part) if sums is None else [a + b for a, b in zip(sums, part)]
        mean_2d_grad, cov_2d_grad, colors_grad, alpha_grad = sums
        # a band's mean2d is the frame's moved by a constant
        RasterizeFunction.last_mean2d_grad = mean_2d_grad.detach()
        mu_g, q_g, s_g, albedo_g, k_j_g, logit_g = crc.backwards_project_sh(
            mean_2d_grad, cov_2d_grad, colors_grad, mu, q, s, cam_rotation, cam_translation,
            ctx.fx, ctx.fy, albedo, k_j, cam_position, alpha_grad, opacity)
        return (mu_g, q_g, s_g, logit_g, albedo_g, k_j_g) + (None,) * 9


def rasterize_bands(gaussians: gaussian, view: dict, band_height: int = 256) -> t.Tensor:
    """The frame [H, W, 3] rendered as bands of ``band_height`` rows (the last
    one shorter when H is not a multiple), opacity as logits like rasterize().
    After backward, ``RasterizeFunction.last_mean2d_grad`` holds the frame's
    dL/d mean2d (the sum over the bands) and ``last_radii2d`` the radii."""
    RasterizeFunction.last_mean2d_grad = None
    RasterizeFunction.last_radii2d = None
    band_rows(int(view["height"]), band_height)  # validates band_height
    return _RasterizeBandsFunction.apply(
        gaussians.mu, gaussians.q, gaussians.s, gaussians.alpha, gaussians.A, gaussians.k_j,
        view["R"], view["T"], view["fx"], view["fy"], view["cx"], view["cy"], view["height"],
        view["width"], band_height)
