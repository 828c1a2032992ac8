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

import importlib
import math

import numpy as np
import pytest
import torch

from gaussian_splatting import synthetic
from gaussian_splatting.rasterizer import RasterizeFunction, rasterize, rasterize_bands
from gaussian_splatting.rasterizer import bands as bands_mod
from gaussian_splatting.rasterizer.bands import (BAND_PAIR_BUDGET, MAX_BAND_PAIRS, band_rows,
                                                  plan_bands)
from helpers import assert_bitwise, assert_grad_close, oracle_forward, scene_arrays
from oracle import oracle as orc
from test_gpu_parity import _np, gpu_forward

pytestmark = pytest.mark.gpu

# the glue module (the package exports its rasterize function under the same name)
glue = importlib.import_module("gaussian_splatting.rasterizer.rasterize")

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


def test_depth_order_is_the_stable_sort_of_the_depth_bits(crc, device):
    """depth_order against numpy's stable argsort of the depths' float bits as
    unsigned: ties (repeated depths), -0.0 / 0.0, negative depths, infinities
    and NaNs of both signs, at a 1024-key partition boundary, beyond 2^18 keys,
    at 2^20 and one beyond (the depth sort's three pass kinds); and keys that
    all share their top byte (the pass over it copies through) up to 2^18
    keys."""
    rng = np.random.default_rng(5)
    for n in (1, 1000, 1024 * 37 + 5, 300_000, 1 << 20, (1 << 20) + 1):
        print(f"[gpu] depth order of {n} keys", flush=True)
        d = np.round(rng.uniform(-2.0, 60.0, n) * 8.0).astype(np.float32) / np.float32(8.0)
        special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 1e-30, -1e30],
                           np.float32)
        k = min(n, 64)
        d[rng.integers(0, n, k)] = special[rng.integers(0, special.size, k)]
        got = _np(crc.depth_order(n, torch.from_numpy(d).to(device)))
        want = np.argsort(d.view(np.uint32), kind="stable").astype(np.int32)
        assert_bitwise(got, want, f"depth order (n={n})")
    # depths in [2, 8): the keys' top byte is the same for all (a pass that
    # copies through), at the largest small-sort size and a partition multiple
    for n in (1024 * 98, 1 << 18):
        print(f"[gpu] depth order of {n} keys in [2, 8)", flush=True)
        d = rng.uniform(2.0, 8.0, n).astype(np.float32)
        d[rng.integers(0, n, 64)] = np.float32(5.0)
        got = _np(crc.depth_order(n, torch.from_numpy(d).to(device)))
        want = np.argsort(d.view(np.uint32), kind="stable").astype(np.int32)
        assert_bitwise(got, want, f"depth order (n={n}, one top byte)")


def test_rasterize_ordered_equals_rasterize(crc, device):
    """Each band of a c5-distribution frame (30k Gaussians, 400x224, 64-row
    bands), rasterized from the frame's depth order, equals rasterize (its own
    depth sort) bit for bit: ids, ranges, n_contrib, image, final T.  The
    depths are quantized so that many Gaussians tie."""
    sc = synthetic.config_scene("c5", requires_grad=False, n=30_000, width=400, height=224)
    a = scene_arrays(sc)
    fw, n = gpu_forward(crc, a, device), a["mu"].shape[0]
    t = fw["tensors"]
    depth = (torch.from_numpy(fw["depth"]).to(device) * 4.0).round() / 4.0
    order = crc.depth_order(n, depth)
    for y0, h in band_rows(a["H"], 64):
        print(f"[gpu] ordered band at row {y0}, {h} rows", flush=True)
        mb = t["mean2d"] - t["mean2d"].new_tensor([0.0, float(y0)])
        args = (depth, mb, t["cov2d"], t["colors"], t["alpha"], h, a["W"])
        want = crc.rasterize(n, *args)
        got = crc.rasterize_ordered(n, order, *args)
        for x, y, nm in zip(got, want, ("img", "sorted_ids", "tile_ranges", "final_T",
                                         "n_contrib")):
            assert_bitwise(_np(x), _np(y), f"{nm} (band {y0})")


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


def _project(crc, g, view):
    n = g.mu.shape[0]
    with torch.no_grad():
        m2, c2, d = crc.project(n, g.mu.detach(), g.q.detach(), g.s.detach(), view["R"],
                                view["T"], view["fx"], view["fy"], view["cx"], view["cy"])
        col = crc.SH(n, (-(view["R"].T @ view["T"])).contiguous(), g.mu.detach(), g.A.detach(),
                     g.k_j.detach())
    return n, m2, c2, d, col


@pytest.mark.parametrize("name,kw", [("c3", dict(n=20_000, width=480, height=272)),
                                     ("c5", dict(n=200_000, width=1000, height=600)),
                                     ("bench", dict())])
def test_tile_row_pairs_count_the_rasterizers_pairs(crc, device, name, kw):
    """Pairs per tile row (the band planner's input) equal the row sums of the
    tile ranges rasterize builds for the whole frame."""
    sc = (synthetic.bench_scene(n=30_000, width=640, height=360, device=device)
          if name == "bench" else synthetic.config_scene(name, device=device, **kw))
    g, view = sc.gaussians, sc.view
    H, W = int(view["height"]), int(view["width"])
    n, m2, c2, d, col = _project(crc, g, view)
    rows = crc.tile_row_pairs(n, m2, c2, H, W).cpu().numpy()
    out = crc.rasterize(n, d, m2, c2, col, torch.sigmoid(g.alpha.detach()), H, W)
    rng = _np(out[2]).reshape(-1, 2).astype(np.int64)
    tx = (W + 15) // 16
    want = (rng[:, 1] - rng[:, 0]).reshape(-1, tx).sum(axis=1)
    assert rows.shape == want.shape and np.array_equal(rows, want)
    assert rows.sum() == out[1].numel()
    empty = crc.tile_row_pairs(0, m2[:0], c2[:0], H, W).cpu().numpy()
    assert empty.shape == want.shape and not empty.any()


def test_planned_bands_equal_the_whole_frame(crc, device):
    """rasterize_bands with its planned bands (a pair budget of a third of the
    frame's pairs: three or four bands) against rasterize: the image bit for
    bit, the gradients within 1e-6 relative."""
    sc = synthetic.config_scene("c3", device=device, n=20_000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    n, m2, c2, d, col = _project(crc, g, view)
    rows = crc.tile_row_pairs(n, m2, c2, 272, 480).cpu().tolist()
    budget = max(max(rows), sum(rows) // 3)
    plan = plan_bands(rows, 272, budget)
    assert len(plan) >= 3
    w = torch.linspace(0.5, 1.5, 480 * 272 * 3, device=device).view(272, 480, 3)

    def run(render):
        for nm in NAMES:
            getattr(g, nm).grad = None
        img = render()
        (img * w).sum().backward()
        return img.detach().clone(), [getattr(g, nm).grad.clone() for nm in NAMES]

    bi, bg = run(lambda: rasterize_bands(g, view, max_pairs=budget))
    wi, wg = run(lambda: rasterize(g, view))
    assert_bitwise(_np(bi), _np(wi), "image")
    for got, want, nm in zip(bg, wg, NAMES):
        err = (got - want).norm() / want.norm().clamp_min(1e-30)
        assert err <= 1e-6, f"d {nm}: {err:.2e}"


def test_tiles_touch_flags_the_gaussians_of_marked_tiles(crc, device):
    """tiles_touch against the oracle's tile rectangles widened by a tile row
    each way, Gaussian by Gaussian, on a seeded mask; every Gaussian the
    rasterizer bins into a marked tile is flagged, whole frame and a band
    rendered from moved means; an empty mask flags none."""
    sc = synthetic.config_scene("c3", device=device, n=20_000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    H, W, ty, tx = 272, 480, 17, 30
    n, m2, c2, d, col = _project(crc, g, view)
    mask = torch.rand(ty, tx, generator=torch.Generator().manual_seed(5)) < 0.1
    got = crc.tiles_touch(n, m2, c2, H, W, mask.to(device)).cpu().numpy()
    _, rect = orc.bin_count(_np(m2), _np(c2), H, W)
    mk = mask.numpy()
    want = np.array([x1 > x0 and bool(mk[max(0, y0 - 1):min(ty, y1 + 1), x0:x1].any())
                     for x0, x1, y0, y1 in rect])
    assert got.dtype == np.bool_ and np.array_equal(got, want)
    op = torch.sigmoid(g.alpha.detach())
    out = crc.rasterize(n, d, m2, c2, col, op, H, W)
    ids, rng = _np(out[1]), _np(out[2]).reshape(-1, 2)
    listed = np.concatenate([ids[a:b] for a, b in rng[mk.reshape(-1)]])
    assert listed.size > 0 and got[listed].all()
    y0, h = 96, 96  # a band: rows 6..11, means moved up by 96
    band = crc.rasterize(n, d, m2 - m2.new_tensor([0.0, 96.0]), c2, col, op, h, W)
    ids_b, rng_b = _np(band[1]), _np(band[2]).reshape(-1, 2)
    listed_b = np.concatenate([ids_b[a:b] for a, b in rng_b[mk[6:12].reshape(-1)]])
    assert listed_b.size > 0 and got[listed_b].all()
    none = crc.tiles_touch(n, m2, c2, H, W, torch.zeros(ty, tx, dtype=torch.bool, device=device))
    assert not none.any()


@pytest.mark.parametrize("order_kind", ["depth_order", "subset"])
def test_tile_skip_leaves_only_the_marked_lists_empty(crc, device, order_kind):
    """rasterize_ordered with tile_skip against the same call without: every
    unmarked tile's list (its ids), image, final T and n_contrib bit for bit,
    every marked tile's range (0, 0) and its pixels blended from nothing (T 1,
    n_contrib 0, black), the lists' total the unmarked tiles' pairs; for the
    frame's depth order and for a subset of the Gaussians in depth order with
    the identity order (as depth-prefix rendering calls it)."""
    sc = synthetic.config_scene("c3", device=device, n=20_000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    H, W, ty, tx = 272, 480, 17, 30
    n, m2, c2, d, col = _project(crc, g, view)
    op = torch.sigmoid(g.alpha.detach())
    order = crc.depth_order(n, d)
    if order_kind == "subset":
        sel = order[::3].long()
        n = int(sel.numel())
        order = torch.arange(n, dtype=torch.int32, device=device)
        m2, c2, d, col, op = m2[sel], c2[sel], d[sel], col[sel], op[sel]
    skip = torch.rand(ty, tx, generator=torch.Generator().manual_seed(7)) < 0.4
    full = crc.rasterize_ordered(n, order, d, m2, c2, col, op, H, W)
    part = crc.rasterize_ordered(n, order, d, m2, c2, col, op, H, W, skip.to(device))
    rf, rp = _np(full[2]).reshape(-1, 2), _np(part[2]).reshape(-1, 2)
    idf, idp = _np(full[1]), _np(part[1])
    sk = skip.numpy().reshape(-1)
    assert (rp[sk] == 0).all()
    for t in np.flatnonzero(~sk):
        assert_bitwise(idp[rp[t, 0]:rp[t, 1]], idf[rf[t, 0]:rf[t, 1]], f"ids of tile {t}")
    assert int((rp[:, 1] - rp[:, 0]).sum()) == int((rf[~sk, 1] - rf[~sk, 0]).sum())
    pix = np.repeat(np.repeat(skip.numpy(), 16, 0), 16, 1)[:H, :W]
    for k, nm in ((0, "image"), (3, "final_T"), (4, "n_contrib")):
        assert_bitwise(_np(part[k])[~pix], _np(full[k])[~pix], nm)
    assert (_np(part[0])[pix] == 0).all() and (_np(part[3])[pix] == 1).all()
    assert (_np(part[4])[pix] == 0).all()


class _TailCapture:
    """Stands in for the extension module: records the four rasterize-backward
    gradients (d mean2d, d cov2d, d colour, d opacity) that the glue hands to
    the fused tail, backwards_project_sh, and calls it."""

    def __init__(self, mod):
        self._mod = mod
        self.last = None

    def __getattr__(self, name):
        return getattr(self._mod, name)

    def backwards_project_sh(self, *args):
        self.last = [args[k].detach().clone() for k in (0, 1, 2, 13)]
        return self._mod.backwards_project_sh(*args)


def test_depth_prefix_equals_the_whole_frame(crc, device, monkeypatch):
    """rasterize_bands in depth-prefix mode (a share of the depth order on the
    whole screen, then the Gaussians of the tiles it left unfinished) against
    rasterize, on c5's distributions at 1M Gaussians and 480x272 (a pixel's
    coverage depends on the Gaussian count, not on the resolution, so tiles
    finish as in c5's full frame), with a seeded N(0, 1) dL/dimage: a prefix of
    0.3 with one band per pass, and 0.1 with an eighth of the frame's pairs as
    the band budget (passes in bands), both passes owning tiles.  The image bit
    for bit rasterize's.  The rasterize-backward gradients the glue hands to
    the fused tail (d mean2d, d cov2d, d colour, d opacity) are the same
    per-(tile, entry) terms summed in another order (the passes' sums added per
    Gaussian): each element within 2e-5 of its sum of |terms| (the oracle's,
    float64) of rasterize's, each tensor within 1e-5 relative.  rasterize's own
    oracle parity is held by the full-size tests."""
    sc = synthetic.config_scene("c5", device=device, n=1_000_000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    a = scene_arrays(sc)
    n, m2, c2, d, col = _project(crc, g, view)
    rows = crc.tile_row_pairs(n, m2, c2, 272, 480).cpu().tolist()
    G = synthetic.grad_image(272, 480, seed=3)
    Gd = G.to(device)
    cap = _TailCapture(glue.crc)
    monkeypatch.setattr(glue, "crc", cap)

    def run(render):
        for nm in NAMES:
            getattr(g, nm).grad = None
        img = render()
        img.backward(Gd)
        torch.cuda.synchronize()
        return img.detach().clone(), [_np(x) for x in cap.last]

    want = oracle_forward(a)
    args = (G.numpy(), want["mean2d"], want["cov2d"], want["colors"], a["alpha"], want["ids"],
            want["ranges"], want["final_T"], want["n_contrib"], 272, 480)
    absum = orc.blend_bwd(*args, with_abs=True)[4:]
    names = ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")

    wi, wb = run(lambda: rasterize(g, view))
    assert np.abs(_np(wi) - want["img"]).max() <= 1e-5
    for prefix, bands in ((0.3, 1), (0.1, 3)):
        budget = BAND_PAIR_BUDGET if bands == 1 else max(max(rows), sum(rows) // 8)
        pi, pb = run(lambda: rasterize_bands(g, view, max_pairs=budget, depth_prefix=prefix))
        st = bands_mod.prefix_stats()
        print(f"[gpu] depth prefix {prefix}: {st}", flush=True)
        assert st["prefix"] == math.ceil(n * prefix)
        assert 0 < st["open_tiles"] < st["tiles"] and st["second_pairs"] > 0
        assert 0 < st["second_gaussians"] < n
        if bands > 1:
            assert st["first_bands"] + st["second_bands"] > 2
        assert_bitwise(_np(pi), _np(wi), f"image (prefix {prefix})")
        for x, y, ab, nm in zip(pb, wb, absum, names):
            x, y = x.reshape(ab.shape).astype(np.float64), y.reshape(ab.shape).astype(np.float64)
            scaled = np.abs(x - y) / np.maximum(ab, 1e-30)
            rel = np.linalg.norm(x - y) / max(np.linalg.norm(y), 1e-30)
            print(f"[gpu] prefix {prefix}: {nm} against rasterize's: relative {rel:.2e}, "
                  f"max |diff| / sum|terms| {scaled.max():.2e}", flush=True)
            assert scaled.max() <= 2e-5 and rel <= 1e-5, nm


def test_backward_accumulate_equals_the_band_sums(crc, device):
    """backwards_rasterization_accumulate (one set of outputs, each band
    added in place) against each band's own backward summed in torch in the
    same order: bit for bit."""
    sc = synthetic.config_scene("c3", device=device, n=20_000, width=480, height=272)
    g, view = sc.gaussians, sc.view
    n, m2, c2, d, col = _project(crc, g, view)
    op = torch.sigmoid(g.alpha.detach())
    G = synthetic.grad_image(272, 480, seed=3).to(device)
    sums, acc = None, None
    for y0, h in band_rows(272, 96):
        mb = m2 - m2.new_tensor([0.0, float(y0)])
        img, ids, rng, fT, nc = crc.rasterize(n, d, mb, c2, col, op, h, 480)
        args = (G[y0:y0 + h], mb, c2, col, op, ids, rng, fT, nc, n, h, 480)
        part = crc.backwards_rasterization_strided(*args)
        sums = [x.clone() for x in part] if sums is None else [a + b for a, b in zip(sums, part)]
        if acc is None:
            acc = [x.clone() for x in part]
        else:
            out = crc.backwards_rasterization_accumulate(*args, acc)
            assert all(o.data_ptr() == a.data_ptr() for o, a in zip(out, acc))
    for a, b, nm in zip(acc, sums, ("mean2d", "cov2d", "colors", "alpha")):
        assert_bitwise(_np(a), _np(b), f"d {nm}")
    with pytest.raises(RuntimeError, match="accumulate_into"):
        crc.backwards_rasterization_accumulate(*args, acc[:3])


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


def test_c5_full_size_in_screen_bands(crc, device, monkeypatch):
    """Config c5 at full size.  The whole frame needs more pairs than int32
    lists hold and is refused; in 256-row bands every band fits and the pairs
    add up to more than 2^31; the pairs per tile row add up to each band's;
    the planned bands are fewer and each within the limit; the frame rendered
    by default (depth-prefix mode) has a finite image in [0, 1] and finite,
    deterministic gradients, and its image is bit for bit the planned bands'
    render of every Gaussian (the rasterize backward's sums within 1e-5
    relative, the parameter gradients within 1e-3)."""
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
    # the planned bands: the same pairs in fewer bands, each within the limit
    # (a band below the first is rasterized from moved means, whose rounding
    # can shift a far-away Gaussian's footprint: its count may differ by a few)
    rows = crc.tile_row_pairs(n, m2, c2, view["height"], view["width"]).cpu().tolist()
    assert sum(rows[:16]) == pairs[0]
    for (y0, h), p in zip(band_rows(view["height"], 256), pairs):
        assert abs(sum(rows[y0 // 16:(y0 + h + 15) // 16]) - p) <= 1e-6 * p
    plan = plan_bands(rows, view["height"])
    planned = [sum(rows[y0 // 16:(y0 + h + 15) // 16]) for y0, h in plan]
    print(f"[gpu] c5 planned bands: {plan}, pairs {planned}", flush=True)
    assert max(planned) <= BAND_PAIR_BUDGET < MAX_BAND_PAIRS and len(plan) < len(pairs)
    del m2, c2, d, col

    cap = _TailCapture(glue.crc)
    monkeypatch.setattr(glue, "crc", cap)

    def frame(depth_prefix=None):
        for nm in NAMES:
            getattr(g, nm).grad = None
        img = rasterize_bands(g, view, depth_prefix=depth_prefix)
        img.sum().backward()
        torch.cuda.synchronize()
        return img.detach(), [getattr(g, nm).grad.clone() for nm in NAMES] + cap.last

    # the default: depth-prefix rendering (the frame needs several bands)
    img, g1 = frame()
    st = bands_mod.prefix_stats()
    print(f"[gpu] c5 depth-prefix frame: {st}", flush=True)
    assert st["prefix"] == math.ceil(n * bands_mod.PREFIX_FRACTION)
    assert st["first_pairs"] + st["second_pairs"] < sum(planned) // 2
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
    del img2, g2
    # every Gaussian in every planned band: the same image bit for bit, the
    # same gradients up to the order of their sums
    print("[gpu] c5 frame in the planned bands without the depth prefix", flush=True)
    img0, g0 = frame(depth_prefix=0.0)
    assert bands_mod.last_stats["prefix"] == 0 and bands_mod.last_stats["bands"] == len(plan)
    assert torch.equal(img, img0)
    blend = ("mean2d", "cov2d", "colors", "alpha (rasterize)")
    for got, want, nm in zip(g1, g0, NAMES + blend):
        err = float((got - want).norm() / want.norm().clamp_min(1e-30))
        print(f"[gpu] c5 d {nm}: prefix vs plain relative error {err:.2e}", flush=True)
        # the rasterize backward's sums within 1e-5; the parameter gradients
        # within 1e-3: a needle-shaped splat's d cov2d cancels to ~1e-6 of its
        # sum of |terms|, so the order of an fp32 sum moves it by up to ~10%,
        # and the projection backward carries that into d q and d s (the
        # tensors differ by ~1e-4 between the two orders of the same terms)
        assert err <= (1e-5 if nm in blend else 1e-3), f"d {nm}: {err:.2e}"
    del img, img0, g1, g0
    torch.cuda.empty_cache()


def _sampled_tiles(rng_np, ranges, tiles_x, count=24):
    """Tiles of a band to hold to the oracle: the first and the last, the four
    longest lists (the backward's long-list mode and split tiles), the tile
    whose list holds each multiple of 2^28 list positions (1 GB of ids) and
    the one before it, then seeded random tiles with entries."""
    T = ranges.shape[0]
    lens = (ranges[:, 1] - ranges[:, 0]).astype(np.int64)
    picked = {0, T - 1}
    picked.update(int(t) for t in np.argsort(-lens, kind="stable")[:4])
    ends = ranges[:, 1].astype(np.int64)
    m = int(ends.max())
    for k in range(1, m // (1 << 28) + 1):
        t = int(np.searchsorted(ends, k << 28, side="right"))
        picked.update(x for x in (t - 1, t) if 0 <= x < T)
    filled = np.flatnonzero(lens > 0)
    while len(picked) < min(count, T) and filled.size:
        picked.add(int(rng_np.choice(filled)))
    return sorted(picked)


def test_c5_full_size_bands_match_the_oracle_on_sampled_tiles(crc, device):
    """Config c5 at full size (5M Gaussians, 3840x2160, 1.1e10 pairs) in its
    planned bands, through the path rasterize_bands takes (the frame's depth
    order, rasterize_ordered per band, the band's backward).  The projection
    and colours are the oracle's bit for bit over all 5M Gaussians.  For each
    band: the pair count equals the oracle's count on the moved means; on
    about 24 sampled tiles per band (the first and last, the longest lists,
    those at each 2^28-entry list boundary, random ones) the tile's ids equal
    the oracle's list built by brute force (every Gaussian whose tile
    rectangle covers the tile, stably ordered by depth bits), and image,
    final T and n_contrib equal the oracle's blend of those lists bit for bit;
    with dL/dimage N(0, 1) on the sampled tiles and zero elsewhere, the
    band's backward (the long-list mode: about 250k entries per tile) is
    within the gradient bar over the same tiles: every element within 1e-4 of
    max(|oracle|, sum|terms|) (or of the fp32 oracle's own distance to
    float64), and each gradient tensor no further from the float64 oracle
    than max(1e-4, 1.5 x the fp32 oracle's own distance).  Both floors are
    wider than the smaller frames' (0.25 sum|terms| and 1e-4 against the fp32
    oracle) because these lists are 100x longer: every term scales with the
    transmittance unwound through the list, and the reference's own fp32
    arithmetic (the fp32 oracle) measures 1e-2 of sum|terms| at the 99.9th
    percentile and up to 6e-2 against float64 on these tiles, and 1e-4 to
    4e-4 per tensor (printed per band)."""
    print("[gpu] c5 full size against the oracle on sampled tiles", flush=True)
    sc = synthetic.config_scene("c5", device=device, requires_grad=False)
    a = scene_arrays(sc)
    n, H, W = a["mu"].shape[0], a["H"], a["W"]
    tiles_x = (W + 15) // 16
    mu, q, s = (torch.from_numpy(a[k]).to(device) for k in ("mu", "q", "s"))
    R, T = torch.from_numpy(a["R"]).to(device), torch.from_numpy(a["t"]).to(device)
    m2, c2, d = crc.project(n, mu, q, s, R, T, a["fx"], a["fy"], a["cx"], a["cy"])
    col = crc.SH(n, torch.from_numpy(a["cam"]).to(device), mu, torch.from_numpy(a["A"]).to(device),
                 torch.from_numpy(a["kj"]).to(device))
    op = torch.from_numpy(a["alpha"]).to(device)
    del mu, q, s
    wm2, wc2, wd = orc.project(a["mu"], a["q"], a["s"], a["R"], a["t"], a["fx"], a["fy"],
                               a["cx"], a["cy"])
    wcol = orc.sh(a["cam"], a["mu"], a["A"], a["kj"])
    assert_bitwise(_np(m2), wm2, "mean2d")
    assert_bitwise(_np(c2), wc2, "cov2d")
    assert_bitwise(_np(d), wd, "depth")
    assert_bitwise(_np(col), wcol, "colors")
    order = crc.depth_order(n, d)
    dbits = wd.view(np.uint32)
    rows = crc.tile_row_pairs(n, m2, c2, H, W).cpu().tolist()
    plan = plan_bands(rows, H)
    print(f"[gpu] c5 bands {plan}", flush=True)
    rng_np = np.random.default_rng(11)
    for y0, h in plan:
        mb = m2 - m2.new_tensor([0.0, float(y0)])
        wmb = (wm2 - np.array([0.0, y0], np.float32)).astype(np.float32)
        img, ids, rng, fT, nc = crc.rasterize_ordered(n, order, d, mb, c2, col, op, h, W)
        counts, rect = orc.bin_count(wmb, wc2, h, W)
        pairs = int(counts.astype(np.int64).sum())
        print(f"[gpu] band rows {y0}..{y0 + h}: {ids.numel()} pairs (oracle {pairs})", flush=True)
        assert ids.numel() == pairs, "band pair count"
        ranges = _np(rng)
        tiles = _sampled_tiles(rng_np, ranges, tiles_x)
        # the oracle's lists of the sampled tiles by brute force
        mini_ids, mini_ranges = [], np.zeros_like(ranges)
        start = 0
        for t in tiles:
            tx, ty = t % tiles_x, t // tiles_x
            cover = np.flatnonzero((rect[:, 0] <= tx) & (tx < rect[:, 1]) & (rect[:, 2] <= ty) &
                                   (ty < rect[:, 3]))
            lst = cover[np.argsort(dbits[cover], kind="stable")].astype(np.int32)
            got = _np(ids[int(ranges[t, 0]):int(ranges[t, 1])])
            assert_bitwise(got, lst, f"ids of tile {t} (band {y0})")
            mini_ids.append(lst)
            mini_ranges[t] = (start, start + lst.size)
            start += lst.size
        mini_ids = np.concatenate(mini_ids) if mini_ids else np.zeros(0, np.int32)
        wimg, wfT, wnc = orc.blend_fwd(mini_ranges, mini_ids, wmb, wc2, wcol, a["alpha"], h, W)
        # the sampled tiles' pixels, bit for bit
        pix = np.zeros((h, W), bool)
        for t in tiles:
            tx, ty = t % tiles_x, t // tiles_x
            pix[ty * 16:ty * 16 + 16, tx * 16:tx * 16 + 16] = True
        assert_bitwise(_np(img)[pix], wimg[pix], f"image (band {y0})")
        assert_bitwise(_np(fT)[pix], wfT[pix], f"final_T (band {y0})")
        assert_bitwise(_np(nc)[pix], wnc[pix], f"n_contrib (band {y0})")
        # the backward with dL/dimage on the sampled tiles only
        G = synthetic.grad_image(h, W, seed=3 + y0).numpy()
        G[~pix] = 0.0
        dm, dc, dcol, dal = crc.backwards_rasterization(
            torch.from_numpy(G).to(device), mb, c2, col, op, ids, rng, fT, nc, n, h, W)
        torch.cuda.synchronize()
        args = (G, wmb, wc2, wcol, a["alpha"], mini_ids, mini_ranges, wfT, wnc, h, W)
        ref = orc.blend_bwd(*args, with_abs=True)
        ref64 = orc.blend_bwd(*args, dtype=np.float64)
        for gg, r, r64, ab, nm in zip((dm, dc, dcol, dal), ref[:4], ref64, ref[4:],
                                      ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
            x = _np(gg).astype(np.float64).reshape(r64.shape)
            rel = lambda u, v: float(np.linalg.norm((u - v).ravel()) /
                                     max(np.linalg.norm(v.ravel()), 1e-300))
            m = ab > 0
            q = lambda u: np.quantile((np.abs(u - r64) / np.maximum(ab, 1e-30))[m], [0.999, 1.0])
            print(f"[gpu] band {y0}: {nm} tensor rel err GPU vs fp64 {rel(x, r64):.2e}, fp32 oracle "
                  f"vs fp64 {rel(r, r64):.2e}, GPU vs fp32 oracle {rel(x, r):.2e}; "
                  f"|x-fp64|/sum|terms| p99.9/max GPU {q(x)} oracle {q(r)}", flush=True)
            worst, tot = assert_grad_close(_np(gg), r, ab, f"band {y0}: {nm}", want64=r64,
                                           floor=1.0, tensor_vs64=True)
            print(f"[gpu] band {y0}: {nm} max scaled error {worst:.2e}", flush=True)
        print(f"[gpu] band {y0}: {len(tiles)} tiles ({mini_ids.size} entries) match", flush=True)
        del img, ids, rng, fT, nc, dm, dc, dcol, dal, mb
        torch.cuda.empty_cache()
