"""Screen bands (gaussian_splatting/rasterizer/bands.py) without a GPU: the band
rows and cameras, and the banded oracle frame against the whole oracle frame."""

from __future__ import annotations

import numpy as np
import pytest

from gaussian_splatting import synthetic
from gaussian_splatting.rasterizer.bands import band_rows, band_views, plan_bands
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


def test_band_rows_cover_the_frame():
    assert band_rows(100, 32) == [(0, 32), (32, 32), (64, 32), (96, 4)]
    assert band_rows(64, 64) == [(0, 64)]
    assert band_rows(0, 16) == []


@pytest.mark.parametrize("name,bh,kw", [("c1", 64, dict()),
                                        ("c3", 48, dict(n=20_000, width=480, height=270))])
def test_banded_oracle_frame_matches_the_whole_frame(orc, name, bh, kw):
    """The oracle frame rendered in bands the way rasterize_bands renders them
    (the frame's projection, means moved up by y0, each band through
    rasterize) and stacked equals the whole frame bit for bit: image, final T
    and n_contrib, and each band's pairs are the frame's pairs of its tile
    rows.  A sign slip in the shift, a wrong band height or a wrong stacking
    order fails it."""
    sc = synthetic.config_scene(name, requires_grad=False, **kw)
    a = scene_arrays(sc)
    whole = oracle_forward(a)
    imgs, ncs, fts, pairs = [], [], [], 0
    for y0, h in band_rows(a["H"], bh):
        mb = (whole["mean2d"] - np.array([0.0, y0], np.float32)).astype(np.float32)
        img, ids, ranges, fT, nc, _ = orc.rasterize(whole["depth"], mb, whole["cov2d"],
                                                    whole["colors"], a["alpha"], h, a["W"])
        imgs.append(img)
        ncs.append(nc)
        fts.append(fT)
        pairs += ids.size
    assert np.array_equal(np.concatenate(imgs), whole["img"])
    assert np.array_equal(np.concatenate(fts), whole["final_T"])
    assert np.array_equal(np.concatenate(ncs), whole["n_contrib"])
    assert pairs == whole["ids"].size
    assert whole["n_contrib"].max() > 0


def _band_pairs(rows, plan):
    return [sum(rows[y0 // 16:(y0 + h + 15) // 16]) for y0, h in plan]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_planned_bands_cover_the_frame_within_the_budget(seed):
    """Planned bands are whole tile rows, contiguous, top to bottom, each
    within the pair budget, as few as the budget allows (the total over the
    budget, rounded up, or one more), and balanced: no band below a third of
    an equal share unless it is the only way to meet the budget."""
    rng = np.random.default_rng(seed)
    H = 2160
    rows = list(rng.integers(0, 2000, size=(H + 15) // 16) * rng.integers(1, 50))
    budget = max(max(rows), sum(rows) // 5)
    plan = plan_bands(rows, H, budget)
    assert plan[0][0] == 0 and sum(h for _, h in plan) == H
    for (a, ha), (b, _) in zip(plan, plan[1:]):
        assert a + ha == b and ha % 16 == 0
    bp = _band_pairs(rows, plan)
    assert sum(bp) == sum(rows) and max(bp) <= budget
    k = -(-sum(rows) // budget)
    assert k <= len(plan) <= k + 1
    assert min(bp) >= sum(rows) / len(plan) / 3


def test_planned_bands_small_cases():
    assert plan_bands([5, 5, 5, 5], 64, 100) == [(0, 64)]
    assert plan_bands([5, 5, 5, 5], 60, 10) == [(0, 32), (32, 28)]
    assert plan_bands([], 0, 10) == []
    assert plan_bands([0, 0, 0], 48, 1) == [(0, 48)]
    # a row over the budget cannot be split
    with pytest.raises(ValueError):
        plan_bands([3, 12, 3], 48, 10)
    # uneven rows: bands cut where the running total reaches its share
    assert _band_pairs([9, 1, 1, 9], plan_bands([9, 1, 1, 9], 64, 12)) == [10, 10]


def test_depth_prefix_rendering_on_the_oracle(orc):
    """Depth-prefix rendering (bands.py) restated on the oracle, end to end: the
    first 30% of the stable depth order (the oracle's own sort of that subset),
    the tiles whose every pixel ends below T = 1e-4 (bands._tile_all), then every
    Gaussian whose oracle tile rectangle, widened by a tile row each way, meets
    an unfinished tile, rendered alone.  Each tile takes the first render's
    outputs if finished, else the second's: image, final T and n_contrib equal
    the whole frame's bit for bit, with tiles of both kinds.  On c5's
    distributions at 1M Gaussians and 480x272 (a pixel's coverage depends on
    the Gaussian count, not on the resolution)."""
    import torch

    from gaussian_splatting.rasterizer.bands import T_MIN, _tile_all

    sc = synthetic.config_scene("c5", requires_grad=False, n=1_000_000, width=480, height=272)
    a = scene_arrays(sc)
    H, W = a["H"], a["W"]
    whole = oracle_forward(a)
    order = np.argsort(whole["depth"].view(np.uint32), kind="stable")

    def render(sel):
        return orc.rasterize(whole["depth"][sel], whole["mean2d"][sel], whole["cov2d"][sel],
                             whole["colors"][sel], a["alpha"][sel], H, W)

    first = render(order[:300_000])
    done = _tile_all(torch.from_numpy(first[3] < np.float32(T_MIN)), H, W).numpy()
    assert 0 < done.sum() < done.size
    _, rect = orc.bin_count(whole["mean2d"], whole["cov2d"], H, W)
    ty, tx = done.shape
    touch = np.array([x1 > x0 and bool((~done)[max(0, y0 - 1):min(ty, y1 + 1), x0:x1].any())
                      for x0, x1, y0, y1 in rect])
    second = render(order[touch[order]])
    own = np.repeat(np.repeat(done, 16, 0), 16, 1)[:H, :W]
    for k, nm in ((0, "image"), (3, "final_T"), (4, "n_contrib")):
        got = np.where(own[..., None] if k == 0 else own, first[k], second[k])
        want = whole["img"] if k == 0 else whole["final_T"] if k == 3 else whole["n_contrib"]
        assert np.array_equal(got, want), nm


def test_depth_prefix_helpers():
    """bands.py's tile helpers: _tile_all (every pixel, pixels beyond the screen
    counted as set), _tile_pixels (the tile set back to a band's pixels),
    _row_runs (runs of set rows), prefix_stats (device counts read as ints)."""
    import torch

    from gaussian_splatting.rasterizer import bands

    m = torch.ones(40, 50, dtype=torch.bool)
    m[17, 33] = False
    want = torch.ones(3, 4, dtype=torch.bool)
    want[1, 2] = False
    assert torch.equal(bands._tile_all(m, 40, 50), want)
    tiles = torch.tensor([[True, False], [False, True], [True, True]])
    pix = bands._tile_pixels(tiles, 16, 20, 20)
    assert pix.shape == (20, 20)
    assert not pix[:16, :16].any() and pix[:16, 16:].all() and pix[16:].all()
    assert bands._row_runs([False, True, True, False, True]) == [(1, 3), (4, 5)]
    assert bands._row_runs([]) == [] and bands._row_runs([True]) == [(0, 1)]
    old = bands.last_stats
    try:
        bands.last_stats = {"prefix": 3, "second_pairs": torch.tensor(7)}
        st = bands.prefix_stats()
        assert st == {"prefix": 3, "second_pairs": 7} and type(st["second_pairs"]) is int
    finally:
        bands.last_stats = old
