"""Screen bands (gaussian_splatting/rasterizer/bands.py) without a GPU: the band
cameras, and the banded oracle frame against the whole oracle frame."""

from __future__ import annotations

import numpy as np
import pytest

from gaussian_splatting import synthetic
from gaussian_splatting.rasterizer.bands import band_views
from helpers import oracle_forward, scene_arrays


def test_band_views_cover_the_frame_top_to_bottom():
    view = dict(R=None, T=None, fx=100.0, fy=100.0, cx=50.0, cy=40.5, height=100, width=64)
    bands = band_views(view, 32)
    assert [y0 for y0, _ in bands] == [0, 32, 64, 96]
    assert [v["height"] for _, v in bands] == [32, 32, 32, 4]
    assert [v["cy"] for _, v in bands] == [40.5, 8.5, -23.5, -55.5]
    for _, v in bands:
        assert v["width"] == 64 and v["cx"] == 50.0 and v["fx"] == 100.0
    assert view["cy"] == 40.5 and view["height"] == 100  # the frame's view is untouched


@pytest.mark.parametrize("h", [0, -16, 8, 17])
def test_band_height_must_be_whole_tiles(h):
    view = dict(cy=8.0, height=64)
    with pytest.raises(ValueError):
        band_views(view, h)


def test_banded_oracle_frame_matches_the_whole_frame(orc):
    """Config c1 rendered by the oracle in 64-row bands (cy - y0, height 64)
    and stacked equals the whole frame: n_contrib identical and the image
    within 1e-5.  A sign slip in the moved principal point, a wrong band
    height or a wrong stacking order fails it."""
    sc = synthetic.config_scene("c1", requires_grad=False)
    a = scene_arrays(sc)
    whole = oracle_forward(a)
    imgs, ncs, fts = [], [], []
    for y0, v in band_views(sc.view, 64):
        b = dict(a, cy=float(v["cy"]), H=int(v["height"]))
        out = oracle_forward(b)
        imgs.append(out["img"])
        ncs.append(out["n_contrib"])
        fts.append(out["final_T"])
    img, nc, ft = np.concatenate(imgs), np.concatenate(ncs), np.concatenate(fts)
    assert img.shape == whole["img"].shape
    assert np.array_equal(nc, whole["n_contrib"])
    assert np.abs(img - whole["img"]).max() <= 1e-5
    assert np.abs(ft - whole["final_T"]).max() <= 1e-5
    assert whole["n_contrib"].max() > 0
