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

Depth-prefix rendering (frames beyond one band, config c5's 1.1e10 pairs):
with hundreds of thousands of entries per tile list, the front-to-back blend
of nearly every tile stops early, once every pixel's T is below 1e-4
(rasterize.cu:264-267), and the rest of its list is never read, yet binning
writes every entry.  So the frame is rendered from two sets of Gaussians:
- first the first ``prefix`` Gaussians of the depth order, on the whole
  screen: each tile's list is then the first part of its full list, in the
  same order, so every pixel's blend takes the same steps as far as it goes;
  a tile whose every pixel stopped (T < 1e-4) is finished, and its image,
  final T, n_contrib and the entries its backward walks ([0, max n_contrib))
  are the full render's, bit for bit;
- then every Gaussian whose tile rectangle (widened by a tile row each way,
  ``tiles_touch``) meets an unfinished tile, on the tile rows that hold one,
  with the finished tiles' lists left empty (``tile_skip``): each unfinished
  tile's list is then its full list.
The image takes each tile from the pass that owns it; each pass's backward
walks only its own tiles (the other pass's tile ranges are emptied), and the
two passes' gradient sums are added per Gaussian.  The image is a full
render's bit for bit; the gradients are the same per-pixel terms summed in
another order.
"""

from __future__ import annotations

import math

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
# Depth-prefix rendering: the share of the depth order the first pass renders
# when rasterize_bands picks the mode itself.
PREFIX_FRACTION = 1.0 / 64
# A pixel's blend stops once T falls below this (rasterize.cu:264-267).
T_MIN = 1e-4
# The last forward's passes, bands and pairs (rasterize_bands; prefix_stats()
# gives them with the device-side counts read back).
last_stats: dict = {}


def prefix_stats() -> dict:
    """last_stats with every count a Python int (device counts are read here,
    not in the forward, so the forward does not wait for its own kernels)."""
    return {k: (int(v) if isinstance(v, t.Tensor) else v) for k, v in last_stats.items()}


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


def _tile_all(mask: t.Tensor, height: int, width: int) -> t.Tensor:
    """[H, W] bool -> [ceil(H/16), ceil(W/16)]: every pixel of the tile set
    (pixels beyond the screen count as set)."""
    ty, tx = (height + TILE - 1) // TILE, (width + TILE - 1) // TILE
    full = mask.new_ones(ty * TILE, tx * TILE)
    full[:height, :width] = mask
    return full.view(ty, TILE, tx, TILE).all(dim=3).all(dim=1)


def _tile_pixels(tiles: t.Tensor, y0: int, h: int, width: int) -> t.Tensor:
    """The [h, W] pixels of rows [y0, y0 + h) (y0 a multiple of 16) that lie in
    a tile set in ``tiles`` [ceil(H/16), ceil(W/16)]."""
    r0, r1 = y0 // TILE, (y0 + h + TILE - 1) // TILE
    rows = tiles[r0:r1].repeat_interleave(TILE, dim=0).repeat_interleave(TILE, dim=1)
    return rows[:h, :width]


def _row_runs(flags) -> list[tuple[int, int]]:
    """[r0, r1) runs of consecutive true entries."""
    runs, r0 = [], None
    for r, f in enumerate(list(flags) + [False]):
        if f and r0 is None:
            r0 = r
        elif not f and r0 is not None:
            runs.append((r0, r))
            r0 = None
    return runs


class _Pass:
    """One set of Gaussians rendered in bands: ``sel`` the Gaussians (frame
    indices in depth order, or None for all of them with the frame's order)
    and per band (y0, h) the rasterize outputs."""

    def __init__(self, sel, rows):
        self.sel, self.rows, self.bands = sel, rows, []


def _render_pass(crc, ps: _Pass, n, order, depths, mean_2d, cov_2d, colors, opacity, width,
                 skip=None):
    """Renders the pass's bands; ``skip`` (the frame's [ceil(H/16), ceil(W/16)]
    bool tiles) marks tiles whose lists may be left empty."""
    if ps.sel is None:
        m, od, dp, mn, cv, cl, op = n, order, depths, mean_2d, cov_2d, colors, opacity
    else:
        # the subset in depth order: its own depth order is the identity
        m = int(ps.sel.numel())
        od = t.arange(m, dtype=t.int32, device=mean_2d.device)
        dp, mn, cv = depths[ps.sel], mean_2d[ps.sel], cov_2d[ps.sel]
        cl, op = colors[ps.sel], opacity[ps.sel]
    for y0, h in ps.rows:
        mean_b = mn - mn.new_tensor([0.0, float(y0)])
        band_skip = None
        if skip is not None:
            r0 = y0 // TILE
            band_skip = skip[r0:r0 + (h + TILE - 1) // TILE].contiguous().view(t.uint8)
        img, ids, ranges, final_T, n_contrib = crc.rasterize_ordered(
            m, od, dp, mean_b, cv, cl, op, h, width, band_skip)
        ps.bands.append([img, mean_b, ids, ranges, final_T, n_contrib])


def _plan_rows(mean_2d, cov_2d, height, width, max_pairs, row_mask=None):
    """Bands over the tile rows of the frame (or over each run of rows set in
    ``row_mask``), planned from the Gaussians' pairs per tile row."""
    rows = frame_row_pairs(mean_2d, cov_2d, height, width)
    if row_mask is None:
        return plan_bands(rows, height, max_pairs)
    out = []
    for r0, r1 in _row_runs(row_mask):
        y0 = r0 * TILE
        for by, bh in plan_bands(rows[r0:r1], min(r1 * TILE, height) - y0, max_pairs):
            out.append((y0 + by, bh))
    return out


def _render_depth_prefix(crc, prefix, n, order, depths, mean_2d, cov_2d, colors, opacity,
                         height, width, max_pairs):
    """The frame from two sets of Gaussians (module docstring, "Depth-prefix
    rendering"): the first ``prefix`` of the depth order on the whole screen,
    then every Gaussian that may reach a tile the first set left unfinished, on
    the tile rows that hold such tiles.  Returns the image, the passes (each
    band's tile ranges emptied on the tiles the other pass owns) and the
    statistics."""
    ty, tx = (height + TILE - 1) // TILE, (width + TILE - 1) // TILE
    first = _Pass(order[:prefix].long(), None)
    first.rows = _plan_rows(mean_2d[first.sel], cov_2d[first.sel], height, width, max_pairs)
    _render_pass(crc, first, n, order, depths, mean_2d, cov_2d, colors, opacity, width)
    image = t.cat([b[0] for b in first.bands], dim=0)
    final_T = t.cat([b[4] for b in first.bands], dim=0)
    # a tile is finished when the blend stopped at every pixel (T < 1e-4): the
    # later Gaussians of its list are never reached
    t_min = t.tensor(T_MIN, dtype=final_T.dtype, device=final_T.device)
    open_tiles = ~_tile_all(final_T < t_min, height, width)
    # one read-back: the unfinished tiles' count, then per tile row whether it holds any
    row_open = open_tiles.any(dim=1)
    counts = t.cat([open_tiles.sum().view(1), row_open.to(t.int64)]).cpu()
    n_open, row_flags = int(counts[0]), counts[1:].bool().tolist()
    stats = {"prefix": int(prefix), "first_bands": len(first.rows),
             "first_pairs": sum(int(b[2].numel()) for b in first.bands),
             "open_tiles": n_open, "tiles": ty * tx,
             "second_gaussians": 0, "second_bands": 0, "second_pairs": 0}
    passes = [first]
    if n_open:
        touch = crc.tiles_touch(n, mean_2d, cov_2d, height, width, open_tiles)
        sel = order[touch[order.long()]].long()
        stats["second_gaussians"] = int(sel.numel())
        if sel.numel():
            second = _Pass(sel, None)
            second.rows = _plan_rows(mean_2d[sel], cov_2d[sel], height, width, max_pairs,
                                     row_flags)
            # the finished tiles' lists stay empty: the second set's Gaussians
            # also cover many of them
            _render_pass(crc, second, n, order, depths, mean_2d, cov_2d, colors, opacity,
                         width, skip=~open_tiles)
            for (y0, h), b in zip(second.rows, second.bands):
                own = _tile_pixels(open_tiles, y0, h, width)
                image[y0:y0 + h] = t.where(own[..., None], b[0], image[y0:y0 + h])
                r0 = y0 // TILE
                b[3].masked_fill_(~open_tiles[r0:r0 + (h + TILE - 1) // TILE].reshape(-1, 1), 0)
            for (y0, h), b in zip(first.rows, first.bands):
                r0 = y0 // TILE
                b[3].masked_fill_(open_tiles[r0:r0 + (h + TILE - 1) // TILE].reshape(-1, 1), 0)
            stats["second_bands"] = len(second.rows)
            # the pairs binned: the lists of the open tiles (sorted_ids keeps
            # the room of every tile the set covers); a device count, read by
            # prefix_stats()
            stats["second_pairs"] = sum((b[3][:, 1] - b[3][:, 0]).sum() for b in second.bands)
            passes.append(second)
    return image, passes, stats


class _RasterizeBandsFunction(t.autograd.Function):
    @staticmethod
    def forward(ctx, mu, q, s, alpha_logits, albedo, k_j, cam_rotation, cam_translation, fx, fy,
                cx, cy, height, width, band_height, max_pairs, depth_prefix):
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
        if depth_prefix is None:
            # automatic: frames beyond one call's pair limit, planned bands
            depth_prefix = PREFIX_FRACTION if band_height is None and len(rows) > 1 else 0.0
        prefix = min(n, max(1, math.ceil(n * depth_prefix))) if depth_prefix > 0 and n else 0
        if prefix:
            image, passes, stats = _render_depth_prefix(
                crc, prefix, n, order, depths, mean_2d, cov_2d, colors, opacity, H, W, max_pairs)
        else:
            whole = _Pass(None, rows)
            _render_pass(crc, whole, n, order, depths, mean_2d, cov_2d, colors, opacity, W)
            image = t.cat([b[0] for b in whole.bands], dim=0)
            passes = [whole]
            stats = {"prefix": 0, "bands": len(rows),
                     "pairs": sum(int(b[2].numel()) for b in whole.bands)}
        global last_stats
        last_stats = stats
        saved = []
        for ps in passes:
            if ps.sel is not None:
                saved.append(ps.sel)
            for b in ps.bands:
                saved += b[1:]
        ctx.save_for_backward(cov_2d, colors, opacity, mu, q, s, albedo, k_j, cam_rotation,
                              cam_translation, cam_position, *saved)
        ctx.passes = [(ps.sel is not None, ps.rows) for ps in passes]
        ctx.n, ctx.W, ctx.fx, ctx.fy = n, W, fx, fy
        return image

    @staticmethod
    def backward(ctx, grad_output):
        crc = glue.crc
        (cov_2d, colors, opacity, mu, q, s, albedo, k_j, cam_rotation, cam_translation,
         cam_position, *saved) = ctx.saved_tensors
        n, W = ctx.n, ctx.W
        sums = None
        k = 0
        for has_sel, rows in ctx.passes:
            sel = None
            if has_sel:
                sel = saved[k]
                k += 1
            m = n if sel is None else int(sel.numel())
            cv = cov_2d if sel is None else cov_2d[sel]
            cl = colors if sel is None else colors[sel]
            op = opacity if sel is None else opacity[sel]
            part = None
            for y0, h in rows:
                mean_b, ids, ranges, final_T, n_contrib = saved[k:k + 5]
                k += 5
                args = (grad_output[y0:y0 + h], mean_b, cv, cl, op, ids, ranges, final_T,
                        n_contrib, m, h, W)
                if part is None:
                    part = list(crc.backwards_rasterization_strided(*args))
                else:
                    # the band's gradients added in place into the running sums
                    crc.backwards_rasterization_accumulate(*args, part)
            if part is None:
                continue
            if sel is None:
                sums = part
            else:
                if sums is None:
                    sums = [x.new_zeros((n,) + tuple(x.shape[1:])) for x in part]
                # each Gaussian of the set once: one add per destination
                for acc, x in zip(sums, part):
                    acc.index_add_(0, sel, x)
        mean_2d_grad, cov_2d_grad, colors_grad, alpha_grad = sums
        # a band's mean2d is the frame's moved by a constant
        RasterizeFunction.last_mean2d_grad = mean_2d_grad.detach()
        mu_g, q_g, s_g, albedo_g, k_j_g, logit_g = crc.backwards_project_sh(
            mean_2d_grad, cov_2d_grad, colors_grad, mu, q, s, cam_rotation, cam_translation,
            ctx.fx, ctx.fy, albedo, k_j, cam_position, alpha_grad, opacity)
        return (mu_g, q_g, s_g, logit_g, albedo_g, k_j_g) + (None,) * 11


def rasterize_bands(gaussians: gaussian, view: dict, band_height: int | None = None,
                    max_pairs: int = BAND_PAIR_BUDGET,
                    depth_prefix: float | None = None) -> t.Tensor:
    """The frame [H, W, 3] rendered as screen bands, opacity as logits like
    rasterize(): bands planned from the frame's pairs per tile row (the fewest
    of at most ``max_pairs`` pairs), or of ``band_height`` rows each (the last
    one shorter when H is not a multiple).  After backward,
    ``RasterizeFunction.last_mean2d_grad`` holds the frame's dL/d mean2d (the
    sum over the bands) and ``last_radii2d`` the radii.

    ``depth_prefix``: the share of the depth order rendered first in
    depth-prefix rendering (module docstring); 0 renders every Gaussian in
    every band; None (default) takes PREFIX_FRACTION for frames that need more
    than one planned band and 0 otherwise.  The image is the same either way;
    the gradients are the same sums in another order.  ``prefix_stats()``
    gives the last forward's passes, bands and pairs."""
    RasterizeFunction.last_mean2d_grad = None
    RasterizeFunction.last_radii2d = None
    if band_height is not None:
        band_rows(int(view["height"]), band_height)  # validates band_height
    if max_pairs <= 0:
        raise ValueError("max_pairs must be positive")
    if depth_prefix is not None and not 0.0 <= float(depth_prefix) <= 1.0:
        raise ValueError(f"depth_prefix must lie in [0, 1], got {depth_prefix}")
    return _RasterizeBandsFunction.apply(
        gaussians.mu, gaussians.q, gaussians.s, gaussians.alpha, gaussians.A, gaussians.k_j,
        view["R"], view["T"], view["fx"], view["fy"], view["cx"], view["cy"], view["height"],
        view["width"], band_height, int(max_pairs),
        None if depth_prefix is None else float(depth_prefix))
