"""Pins of the oracle's alpha blend forward/backward (rasterize.cu:168-281,
rasterize_backward.cu:6-236) and of the whole pipeline against closed forms, a
brute-force per-pixel loop and finite differences (the reference's gradcheck scenes)."""

import math

import numpy as np


def _render(orc, mean2d, cov2d, colors, alpha, depth, H, W, dtype=np.float32):
    """Bin/sort in fp32 (discrete), blend in `dtype`."""
    m32, c32, d32 = (np.asarray(a, np.float32) for a in (mean2d, cov2d, depth))
    keys, ids = orc.emit_keys(m32, c32, d32, H, W)
    skeys, sids = orc.sort_pairs(keys, ids)
    ranges = orc.tile_ranges(skeys, orc.tiles(H, W))
    img, fT, nc = orc.blend_fwd(ranges, sids, mean2d, cov2d, colors, alpha, H, W, dtype=dtype)
    return img, fT, nc, sids, ranges


def test_isotropic_single_gaussian_closed_form(orc):
    """tests/test_cuda_backward.py:164-219 scene: mean (8,8), cov (4,0,4), colour
    (.25,.45,.70), opacity 0.6 on a 16x16 tile: conic (1/4, 0, 1/4), so
    alpha = min(.99, .6 exp(-((x-8)^2 + (y-8)^2)/8)), img = colour alpha where
    alpha >= 1/255, final_T = 1 - alpha, n_contrib = 1 there and 0 elsewhere."""
    mean = np.array([[8.0, 8.0]], np.float32)
    cov = np.array([[4.0, 0.0, 4.0]], np.float32)
    col = np.array([[0.25, 0.45, 0.70]], np.float32)
    op = np.array([0.6], np.float32)
    img, fT, nc, sids, ranges = _render(orc, mean, cov, col, op, [2.0], 16, 16)
    assert list(ranges[0]) == [0, 1] and list(sids) == [0]
    y, x = np.mgrid[0:16, 0:16].astype(np.float64)
    a = np.minimum(0.99, 0.6 * np.exp(-((x - 8) ** 2 + (y - 8) ** 2) / 8.0))
    on = a >= 1 / 255
    np.testing.assert_array_equal(nc, on.astype(np.int32))
    np.testing.assert_allclose(img, np.where(on[..., None], a[..., None] * col[0], 0), atol=2e-7)
    np.testing.assert_allclose(fT, np.where(on, 1 - a, 1), atol=2e-7)


def _brute_blend(mean, cov, col, op, order, H, W):
    """Per-pixel loop in float64 over the depth-ordered Gaussians touching each tile."""
    img = np.zeros((H, W, 3))
    fT = np.ones((H, W))
    nc = np.zeros((H, W), np.int64)
    for py in range(H):
        for px in range(W):
            T, C, cnt, last = 1.0, np.zeros(3), 0, 0
            for g in order[(py // 16, px // 16)]:
                cnt += 1
                a_, b_, c_ = cov[g]
                det = a_ * c_ - b_ * b_
                inv = 1 / det if det > 0 else 0.0
                cx, cy, cz = c_ * inv, -b_ * inv, a_ * inv
                dx, dy = px - mean[g, 0], py - mean[g, 1]
                power = -0.5 * (cx * dx * dx + 2 * cy * dx * dy + cz * dy * dy)
                if power > 0:
                    continue
                al = min(0.99, op[g] * math.exp(power))
                if al < np.float32(1 / 255):
                    continue
                C += col[g] * al * T
                T *= 1 - al
                last = cnt
                if T < np.float32(1e-4):
                    break
            img[py, px], fT[py, px], nc[py, px] = C, T, last
    return img, fT, nc


def test_multi_gaussian_matches_brute_force(orc):
    rng = np.random.default_rng(0)
    H, W, n = 40, 48, 220
    mean = np.c_[rng.uniform(-5, W + 5, n), rng.uniform(-5, H + 5, n)].astype(np.float32).astype(np.float64)
    L = rng.normal(0, 1, (n, 2, 2)) * rng.uniform(1, 5, (n, 1, 1))
    C = L @ np.transpose(L, (0, 2, 1))
    cov = np.c_[C[:, 0, 0] + 0.3, C[:, 0, 1], C[:, 1, 1] + 0.3].astype(np.float32).astype(np.float64)
    col = rng.uniform(0, 1, (n, 3))
    op = rng.uniform(0.6, 0.99, n)
    depth = rng.uniform(1, 5, n).astype(np.float32)
    img, fT, nc, sids, ranges = _render(orc, mean, cov, col, op, depth, H, W, dtype=np.float64)
    tiles_x = (W + 15) // 16
    order = {}
    for t in range(len(ranges)):
        order[(t // tiles_x, t % tiles_x)] = sids[ranges[t, 0]:ranges[t, 1]]
    # the list order itself: ascending depth, ties by id, per tile
    for lst in order.values():
        d = depth[lst]
        assert np.all((d[:-1] < d[1:]) | ((d[:-1] == d[1:]) & (lst[:-1] < lst[1:])))
    bi, bT, bn = _brute_blend(mean, cov, col, op, order, H, W)
    np.testing.assert_array_equal(nc, bn)
    np.testing.assert_allclose(img, bi, atol=1e-12)
    np.testing.assert_allclose(fT, bT, atol=1e-12)
    assert (nc > 0).mean() > 0.5 and (fT < 1e-4).any()  # the scene exercises early stop


def _smooth_scene(rng, n=12, H=32, W=32):
    mean = np.c_[rng.uniform(4, W - 4, n), rng.uniform(4, H - 4, n)]
    L = rng.normal(0, 1, (n, 2, 2)) * rng.uniform(1.5, 3, (n, 1, 1))
    C = L @ np.transpose(L, (0, 2, 1))
    cov = np.c_[C[:, 0, 0] + 1.0, C[:, 0, 1], C[:, 1, 1] + 1.0]
    col = rng.uniform(0.1, 0.9, (n, 3))
    op = rng.uniform(0.2, 0.6, n)
    depth = rng.uniform(1, 5, n)
    return mean, cov, col, op, depth


def test_blend_backward_matches_finite_differences_fp64(orc):
    rng = np.random.default_rng(1)
    H = W = 32
    mean, cov, col, op, depth = _smooth_scene(rng)
    G = rng.normal(size=(H, W, 3))
    img, fT, nc, sids, ranges = _render(orc, mean, cov, col, op, depth, H, W, dtype=np.float64)
    dm, dc, dcol, dop = orc.blend_bwd(G, mean, cov, col, op, sids, ranges, fT, nc, H, W,
                                      dtype=np.float64)
    base = {"mean": mean, "cov": cov, "col": col, "op": op}
    got = {"mean": dm, "cov": dc, "col": dcol, "op": dop[:, 0]}
    eps = 1e-7
    for name, x in base.items():
        num = np.zeros_like(x)
        for idx in np.ndindex(*x.shape):
            v = []
            for sgn in (1, -1):
                args = {k: a.copy() for k, a in base.items()}
                args[name][idx] += sgn * eps
                # same tile lists (binning is discrete); only the blend is differenced
                im, _, _ = orc.blend_fwd(ranges, sids, args["mean"], args["cov"], args["col"],
                                         args["op"], H, W, dtype=np.float64)
                v.append(np.sum(G * im))
            num[idx] = (v[0] - v[1]) / (2 * eps)
        np.testing.assert_allclose(got[name], num, rtol=2e-5, atol=2e-6 * np.abs(num).max(),
                                   err_msg=name)


def test_blend_backward_fp32_terms_match_fp64(orc):
    """fp32 per-pixel terms accumulated in float64 vs the float64 oracle (same lists)."""
    rng = np.random.default_rng(2)
    H = W = 32
    mean, cov, col, op, depth = _smooth_scene(rng)
    args32 = [np.asarray(a, np.float32) for a in (mean, cov, col, op)]
    G = rng.normal(size=(H, W, 3)).astype(np.float32)
    img, fT, nc, sids, ranges = _render(orc, *args32, depth, H, W)
    g32 = orc.blend_bwd(G, *args32, sids, ranges, fT, nc, H, W)
    img64, fT64, nc64, _, _ = _render(orc, *[a.astype(np.float64) for a in args32], depth, H, W,
                                      dtype=np.float64)
    assert np.array_equal(nc, nc64)
    g64 = orc.blend_bwd(G.astype(np.float64), *[a.astype(np.float64) for a in args32], sids, ranges,
                        fT64, nc64, H, W, dtype=np.float64)
    for a, b in zip(g32, g64):
        np.testing.assert_allclose(a, b, rtol=1e-3, atol=1e-5 * np.abs(b).max())


def _pipeline(orc, mu, q, s, op, A, kj, R, t, cam, H, W, dtype):
    fx, fy, cx, cy = cam
    m2, c2, d = orc.project(mu, q, s, R, t, fx, fy, cx, cy, dtype=dtype)
    campos = -(np.asarray(R, np.float64).T @ np.asarray(t, np.float64))
    col = orc.sh(campos, mu, A, kj, dtype=dtype)
    return m2, c2, d, col


def test_reference_full_pipeline_gradcheck_scene(orc):
    """tests/test_cuda_backward.py:222-263: one Gaussian at mu (.05,-.04,4), fx=fy=16,
    cx=cy=8 on a 16x16 image, loss = sum of pixels [7:9, 7:9]; the chained fp32 oracle
    backward against central differences of the float64 forward (reference tolerances)."""
    H = W = 16
    R, t = np.eye(3), np.zeros(3)
    cam = (16.0, 16.0, 8.0, 8.0)
    quat = np.array([1.0, 0.1, -0.05, 0.02], np.float32)
    quat = quat / np.linalg.norm(quat)
    inputs = {
        "mu": np.array([[0.05, -0.04, 4.0]], np.float32),
        "q": quat.reshape(1, 4).astype(np.float32),
        "s": np.full((1, 3), -2.0, np.float32),
        "op": np.array([0.5], np.float32),
        "A": np.zeros((1, 3), np.float32),
        "kj": np.linspace(-0.005, 0.005, 45, dtype=np.float32).reshape(1, 15, 3),
    }
    Gimg = np.zeros((H, W, 3), np.float32)
    Gimg[7:9, 7:9] = 1.0

    def loss64(p):
        m2, c2, d, col = _pipeline(orc, p["mu"], p["q"], p["s"], p["op"], p["A"], p["kj"], R, t,
                                   cam, H, W, np.float64)
        img, _, _, _, _ = _render(orc, m2, c2, col, p["op"], d, H, W, dtype=np.float64)
        return float(np.sum(Gimg * img))

    # analytic, fp32 chain: blend -> SH -> projection (rasterize.py:76-134)
    p32 = inputs
    m2, c2, d, col = _pipeline(orc, p32["mu"], p32["q"], p32["s"], p32["op"], p32["A"], p32["kj"],
                               R, t, cam, H, W, np.float32)
    img, fT, nc, sids, ranges = _render(orc, m2, c2, col, p32["op"], d, H, W)
    assert float(np.sum(Gimg * img)) > 1e-3
    dm, dc, dcol, dop = (np.asarray(x, np.float32) for x in
                         orc.blend_bwd(Gimg, m2, c2, col, p32["op"], sids, ranges, fT, nc, H, W))
    dA, dkj, dmu_sh = orc.sh_bwd(dcol, p32["mu"], p32["A"], p32["kj"], np.zeros(3))
    dmu, dq, ds = orc.project_bwd(dm, dc, p32["mu"], p32["q"], p32["s"], R, t, *cam)
    got = {"mu": dmu + dmu_sh, "q": dq, "s": ds, "op": dop[:, 0], "A": dA, "kj": dkj}
    for name, x in inputs.items():
        num = np.zeros(x.shape)
        for idx in np.ndindex(*x.shape):
            v = []
            for sgn in (1, -1):
                p = {k: a.astype(np.float64) for k, a in inputs.items()}
                p[name][idx] += sgn * 1e-3
                v.append(loss64(p))
            num[idx] = (v[0] - v[1]) / 2e-3
        assert np.all(np.abs(got[name] - num) <= 1e-3 + 1e-2 * np.abs(num)), (name, got[name], num)


def test_reference_rasterize_gradcheck_scene(orc):
    """tests/test_cuda_backward.py:164-219: d(sum img[6:10, 6:10]) / d(mean2d, cov2d,
    colour, opacity) for the isotropic Gaussian, fp32 analytic vs float64 differences."""
    H = W = 16
    inputs = {"mean": np.array([[8.0, 8.0]], np.float32), "cov": np.array([[4.0, 0.0, 4.0]], np.float32),
              "col": np.array([[0.25, 0.45, 0.70]], np.float32), "op": np.array([0.6], np.float32)}
    Gimg = np.zeros((H, W, 3), np.float32)
    Gimg[6:10, 6:10] = 1.0
    img, fT, nc, sids, ranges = _render(orc, inputs["mean"], inputs["cov"], inputs["col"],
                                        inputs["op"], [2.0], H, W)
    assert float(np.sum(Gimg * img)) > 1e-2
    dm, dc, dcol, dop = orc.blend_bwd(Gimg, inputs["mean"], inputs["cov"], inputs["col"],
                                      inputs["op"], sids, ranges, fT, nc, H, W)
    got = {"mean": dm, "cov": dc, "col": dcol, "op": dop[:, 0]}
    for name, x in inputs.items():
        num = np.zeros(x.shape)
        for idx in np.ndindex(*x.shape):
            v = []
            for sgn in (1, -1):
                p = {k: a.astype(np.float64) for k, a in inputs.items()}
                p[name][idx] += sgn * 1e-3
                im, _, _ = orc.blend_fwd(ranges, sids, p["mean"], p["cov"], p["col"], p["op"], H, W,
                                         dtype=np.float64)
                v.append(np.sum(Gimg * im))
            num[idx] = (v[0] - v[1]) / 2e-3
        assert np.all(np.abs(got[name] - num) <= 1e-3 + 1e-2 * np.abs(num)), (name, got[name], num)
