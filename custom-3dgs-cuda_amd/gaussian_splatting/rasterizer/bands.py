"""Screen-band rendering: frames whose (Gaussian, tile) pair count is beyond the
int32 lists of the rasterize surface (the reference keeps the pair count, the
offsets and ``sorted_ids`` in int, rasterize.cu:382-390, rasterize.h:7-8).

One autograd Function renders the frame as bands of whole tile rows:
- forward: the fused head (camera position, project, radii, SH, sigmoid) and
  the depth sort run once; each band of rows [y0, y0 + h) is rasterized from
  the frame's projection and depth order with the means moved up by y0 rows;
- backward: each band's rasterize backward reads its rows of dL/dimage in
  place and adds its d mean2d, d cov2d, d colour and d opacity into the
  frame's (the first band writes them), and the fused tail (SH and
  projection backward, the sigmoid's backward) runs once.

Bands are whole tile rows (heights multiples of the 16-pixel tile), so a
band's tiles are the frame's tiles.  By default the rows are planned from the
frame's pairs per tile row (``custom_rasterizer_cuda.tile_row_pairs``, counted
as the rasterizer counts them): as few bands as the int32 pair limit allows,
balanced in pairs, so that each launch has as many tiles as possible; a fixed
``band_height`` is also accepted.  Moving a mean by a whole number of rows is exact in fp32
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
# The rasterize surface's pair limit per call (GSR_ERR_TOO_MANY_PAIRS beyond):
# 2^31 - 2^16, the int32 lists less the headroom of in-kernel list arithmetic.
MAX_BAND_PAIRS = 2**31 - 2**16
# The planner's default budget per band: the limit less 1/128.  A band below
# the first is rasterized from means moved up by its first row, and a mean far
# above the band can round in its last bit and shift that Gaussian's footprint
# by a tile, so a band's own pair count can differ slightly from the sum of
# the frame's rows it covers (by about 1e-8 of the pairs at config c5).
BAND_PAIR_BUDGET = MAX_BAND_PAIRS - (MAX_BAND_PAIRS >> 7)


def plan_bands(row_pairs, height: int, max_pairs: int = BAND_PAIR_BUDGET) -> list[tuple[int, int]]:
    """(y0, h) bands of whole tile rows for a frame whose tile row r holds
    ``row_pairs[r]`` pairs: the fewest bands of at most ``max_pairs`` pairs each,
    cut near equal shares of the frame's pairs."""
    rows = [int(x) for x in row_pairs]
    if height <= 0 or not rows:
        return []
    if max(rows) > max_pairs:
        raise ValueError(f"a tile row holds {max(rows)} pairs, more than a band may "
                         f"({max_pairs})")
    total = sum(rows)
    k = max(1, -(-total // max_pairs))
    while True:
        cuts, acc, band, i = [0], 0, 0, 1
        for r, c in enumerate(rows):
            # close the band before this row when it would overflow, or when the
            # band has reached its share of the frame
            if band and (band + c > max_pairs or (i < k and acc >= total * i / k)):
                cuts.append(r)
                band = 0
                i += 1
            acc += c
            band += c
        cuts.append(len(rows))
        if len(cuts) - 1 <= k:
            break
        k += 1
    out = []
    for r0, r1 in zip(cuts[:-1], cuts[1:]):
        y0 = r0 * TILE
        out.append((y0, min((r1 - r0) * TILE, height - y0)))
    return out


def frame_row_pairs(mean_2d: t.Tensor, cov_2d: t.Tensor, height: int, width: int) -> list[int]:
    """Pairs per tile row of the frame, from its projected means and covariances."""
    crc = glue.crc
    if crc is None:
        raise ImportError("custom_rasterizer_cuda is not built. "
                          "Build it with: python custom-3dgs-cuda_amd/build.py")
    n = int(mean_2d.shape[0])
    return crc.tile_row_pairs(n, mean_2d.contiguous(), cov_2d.contiguous(), int(height),
                              int(width)).cpu().tolist()


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
                cx, cy, height, width, band_height, max_pairs):
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
        if band_height is None:
            rows = plan_bands(frame_row_pairs(mean_2d, cov_2d, H, W), H, max_pairs)
        else:
            rows = band_rows(H, band_height)
        # one depth order for all bands: each band's visible Gaussians appear
        # in it as that band's own depth sort would order them
        order = crc.depth_order(n, depths)
        images, saved = [], []
        for y0, h in rows:
            mean_b = mean_2d - mean_2d.new_tensor([0.0, float(y0)])
            img, ids, ranges, final_T, n_contrib = crc.rasterize_ordered(
                n, order, depths, mean_b, cov_2d, colors, opacity, h, W)
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
            args = (grad_output[y0:y0 + h], mean_b, cov_2d, colors, opacity, ids, ranges,
                    final_T, n_contrib, n, h, W)
            if sums is None:
                sums = list(crc.backwards_rasterization_strided(*args))
            else:
                # the band's gradients added in place into the running sums
                crc.backwards_rasterization_accumulate(*args, sums)
        mean_2d_grad, cov_2d_grad, colors_grad, alpha_grad = sums
        # a band's mean2d is the frame's moved by a constant
        RasterizeFunction.last_mean2d_grad = mean_2d_grad.detach()
        mu_g, q_g, s_g, albedo_g, k_j_g, logit_g = crc.backwards_project_sh(
            mean_2d_grad, cov_2d_grad, colors_grad, mu, q, s, cam_rotation, cam_translation,
            ctx.fx, ctx.fy, albedo, k_j, cam_position, alpha_grad, opacity)
        return (mu_g, q_g, s_g, logit_g, albedo_g, k_j_g) + (None,) * 10


def rasterize_bands(gaussians: gaussian, view: dict, band_height: int | None = None,
                    max_pairs: int = BAND_PAIR_BUDGET) -> t.Tensor:
    """The frame [H, W, 3] rendered as screen bands, opacity as logits like
    rasterize(): bands planned from the frame's pairs per tile row (the fewest
    of at most ``max_pairs`` pairs), or of ``band_height`` rows each (the last
    one shorter when H is not a multiple).  After backward,
    ``RasterizeFunction.last_mean2d_grad`` holds the frame's dL/d mean2d (the
    sum over the bands) and ``last_radii2d`` the radii."""
    RasterizeFunction.last_mean2d_grad = None
    RasterizeFunction.last_radii2d = None
    if band_height is not None:
        band_rows(int(view["height"]), band_height)  # validates band_height
    if max_pairs <= 0:
        raise ValueError("max_pairs must be positive")
    return _RasterizeBandsFunction.apply(
        gaussians.mu, gaussians.q, gaussians.s, gaussians.alpha, gaussians.A, gaussians.k_j,
        view["R"], view["T"], view["fx"], view["fy"], view["cx"], view["cy"], view["height"],
        view["width"], band_height, int(max_pairs))
