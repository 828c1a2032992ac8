"""Pins of the oracle's binning, key emission, sort and tile ranges
(rasterize.cu:7-166) against brute force, numpy's stable sort and closed forms."""

import numpy as np


def _random_splats(rng, n, W, H):
    mean = np.c_[rng.uniform(-40, W + 40, n), rng.uniform(-40, H + 40, n)].astype(np.float32)
    L = rng.normal(0, 1, (n, 2, 2)) * rng.uniform(0.5, 12, (n, 1, 1))
    cov = L @ np.transpose(L, (0, 2, 1))
    cov = np.c_[cov[:, 0, 0] + 0.3, cov[:, 0, 1], cov[:, 1, 1] + 0.3].astype(np.float32)
    depth = rng.uniform(0.3, 10, n).astype(np.float32)
    return mean, cov, depth


def _rect64(mean, cov, W, H):
    """Closed-form rectangle in float64: radius = ceil(3 sqrt(mid + sqrt(max(0.1,
    ((a-c)/2)^2 + b^2)))), pixel box clamped to the screen, tiles touching it."""
    a, b, c = cov.astype(np.float64).T
    lam = 0.5 * (a + c) + np.sqrt(np.maximum(0.1, (0.5 * (a - c)) ** 2 + b * b))
    r3 = 3 * np.sqrt(lam)
    r = np.ceil(r3)
    x0 = np.maximum(0, np.floor(mean[:, 0] - r)).astype(np.int64)
    x1 = np.minimum(W, np.ceil(mean[:, 0] + r)).astype(np.int64)
    y0 = np.maximum(0, np.floor(mean[:, 1] - r)).astype(np.int64)
    y1 = np.minimum(H, np.ceil(mean[:, 1] + r)).astype(np.int64)
    near_int = np.abs(r3 - np.round(r3)) < 1e-4
    return x0, x1, y0, y1, near_int


def test_counts_match_brute_force_tile_enumeration(orc):
    rng = np.random.default_rng(0)
    W, H = 200, 136
    mean, cov, _ = _random_splats(rng, 3000, W, H)
    counts, rect = orc.bin_count(mean, cov, H, W)
    x0, x1, y0, y1, near = _rect64(mean, cov, W, H)
    tx, ty = (W + 15) // 16, (H + 15) // 16
    checked = 0
    for i in range(len(mean)):
        if near[i] or x1[i] <= x0[i] or y1[i] <= y0[i]:
            continue
        # every tile whose 16x16 pixel square meets the (non-empty) pixel box
        want = sum(1 for yy in range(ty) for xx in range(tx)
                   if 16 * xx < x1[i] and 16 * xx + 16 > x0[i] and 16 * yy < y1[i] and 16 * yy + 16 > y0[i])
        assert counts[i] == want, i
        checked += 1
    assert checked > 2000


def test_degenerate_and_saturating_rectangles(orc):
    W, H = 20, 40
    mean = np.array([
        [30.0, 10.0],    # right of a 20-wide screen whose last tile is partial
        [5.0, 5.0],      # det <= 0
        [10.0, 10.0],    # huge covariance: radius saturates -> whole screen
        [np.nan, 5.0],   # NaN mean: the casts give 0 -> no tiles
    ], np.float32)
    cov = np.array([[4, 0, 4], [1, 2, 1], [1e38, 0, 1e38], [4, 0, 4]], np.float32)
    counts, rect = orc.bin_count(mean, cov, H, W)
    # radius ceil(3*sqrt(4+sqrt(.1))) = 7: x box [23, 20) is empty, but the tile
    # arithmetic gives [23//16, (20+15)//16) = [1, 2): one tile (rasterize.cu:48-59)
    assert counts[0] == 1 * 2
    assert counts[1] == 0
    assert counts[2] == ((W + 15) // 16) * ((H + 15) // 16)
    assert counts[3] == 0


def test_emission_sort_and_ranges(orc):
    rng = np.random.default_rng(1)
    W, H = 160, 96
    mean, cov, depth = _random_splats(rng, 800, W, H)
    depth[::7] = depth[3]  # depth ties: order must fall back to Gaussian id
    keys, ids = orc.emit_keys(mean, cov, depth, H, W)
    counts, rect = orc.bin_count(mean, cov, H, W)
    assert keys.size == counts.sum()
    # Gaussian-major, ty outer / tx inner (rasterize.cu:124-135)
    off = np.concatenate([[0], np.cumsum(counts)])
    tiles_x = (W + 15) // 16
    for g in rng.choice(len(mean), 50, replace=False):
        x0, x1, y0, y1 = rect[g]
        want = [(ty * tiles_x + tx) for ty in range(y0, y1) for tx in range(x0, x1)]
        got = keys[off[g]:off[g + 1]] >> np.uint64(32)
        assert list(got) == want
        assert np.all(ids[off[g]:off[g + 1]] == g)
        assert np.all((keys[off[g]:off[g + 1]] & np.uint64(0xffffffff)) == depth[g:g + 1].view(np.uint32)[0])
    skeys, sids = orc.sort_pairs(keys, ids)
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(skeys, keys[order])
    np.testing.assert_array_equal(sids, ids[order])
    T = tiles_x * ((H + 15) // 16)
    ranges = orc.tile_ranges(skeys, T)
    hi = (skeys >> np.uint64(32)).astype(np.int64)
    lo_b = np.searchsorted(hi, np.arange(T), "left")
    hi_b = np.searchsorted(hi, np.arange(T), "right")
    empty = lo_b == hi_b
    np.testing.assert_array_equal(ranges[~empty, 0], lo_b[~empty])
    np.testing.assert_array_equal(ranges[~empty, 1], hi_b[~empty])
    assert np.all(ranges[empty] == 0)


def test_depth_presort_then_tile_sort_equals_full_key_sort(orc):
    """The HIP path orders pairs by a stable depth sort of the Gaussians, emission in
    that order, then a stable sort on the tile id alone; this is the same order as the
    reference's stable sort of all 64 key bits over Gaussian-major emission."""
    rng = np.random.default_rng(2)
    W, H = 256, 144
    mean, cov, depth = _random_splats(rng, 1500, W, H)
    depth[rng.choice(1500, 400)] = np.float32(2.5)
    keys, ids = orc.emit_keys(mean, cov, depth, H, W)
    _, want_ids = orc.sort_pairs(keys, ids)
    counts, rect = orc.bin_count(mean, cov, H, W)
    dkey = np.where(counts > 0, depth.view(np.uint32), np.uint32(0xffffffff))
    perm = np.argsort(dkey, kind="stable")
    tiles_x = (W + 15) // 16
    t_list, g_list = [], []
    for g in perm:
        x0, x1, y0, y1 = rect[g]
        for ty in range(y0, y1):
            for tx in range(x0, x1):
                t_list.append(ty * tiles_x + tx)
                g_list.append(g)
    t_arr, g_arr = np.array(t_list), np.array(g_list)
    got_ids = g_arr[np.argsort(t_arr, kind="stable")]
    np.testing.assert_array_equal(got_ids, want_ids)
