"""Screen-band rendering: frames whose (Gaussian, tile) pair count is beyond the
int32 lists of the rasterize surface (the reference keeps the pair count, the
offsets and ``sorted_ids`` in int, rasterize.cu:382-390, rasterize.h:7-8).

A band of rows [y0, y0 + h) is rendered through the unchanged surface as a
frame of its own: the same camera with the principal point moved up by y0
(cy - y0) and height h, so each Gaussian's mean lands y0 rows higher and the
band's pixel (x, y) sees what the frame's pixel (x, y0 + y) sees.  Band heights
are multiples of the 16-pixel tile, so a band's tiles are the frame's tiles.
The band images are stacked; autograd sums every band's gradients into the
shared parameters.

The banded image equals the frame's up to the rounding of the moved mean:
(f_y y / z + (c_y - y_0)) and (f_y y / z + c_y) - y_0 differ in the last bit,
which can flip an alpha or saturation threshold at a pixel.  Each band is
itself rendered exactly (bit for bit the reference's math on that band's
camera).
"""

from __future__ import annotations

import torch as t

from gaussian_splatting.rasterizer.rasterize import RasterizeFunction, rasterize
from gaussian_splatting.scene.gaussian import gaussian

TILE = 16


def band_views(view: dict, band_height: int) -> list[tuple[int, dict]]:
    """(y0, view of rows [y0, y0 + h)) for each band, top to bottom."""
    if band_height <= 0 or band_height % TILE:
        raise ValueError(f"band_height must be a positive multiple of {TILE}, got {band_height}")
    H = int(view["height"])
    out = []
    for y0 in range(0, H, band_height):
        v = dict(view)
        v["cy"] = float(view["cy"]) - y0
        v["height"] = min(band_height, H - y0)
        out.append((y0, v))
    return out


def rasterize_bands(gaussians: gaussian, view: dict, band_height: int = 128) -> t.Tensor:
    """The frame [H, W, 3] rendered as bands of ``band_height`` rows (the last
    one shorter when H is not a multiple).  After backward,
    ``RasterizeFunction.last_mean2d_grad`` holds the sum over the bands of
    dL/d mean2d (a band's mean2d is the frame's moved by a constant)."""
    images = []
    RasterizeFunction.band_accumulate = True
    try:
        for _, v in band_views(view, band_height):
            images.append(rasterize(gaussians, v))
    finally:
        RasterizeFunction.band_accumulate = False
    RasterizeFunction.last_mean2d_grad = None
    return t.cat(images, dim=0)
