"""GPU parity: the HIP library (through custom_rasterizer_cuda) against the CPU oracle.

Bars (rasterizer baseline): sorted keys, sorted ids, tile ranges and n_contrib
bit-exact; fp32 images and final transmittance within 1e-5 absolute; gradients
within 1e-4 relative (helpers.assert_grad_close: 1e-4 of |oracle|, floored at
5e-6 of the sum of |terms| for sums that cancel).  Projection, SH, images and
transmittance are also checked bit for bit, which the shared operation order
makes the expected outcome.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splatting import synthetic
from helpers import assert_bitwise, assert_grad_close, oracle_forward, scene_arrays
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _dev(a, device, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)


def _np(t):
    return t.detach().cpu().numpy()


def gpu_forward(crc, a: dict, device) -> dict:
    n = a["mu"].shape[0]
    mu, q, s = _dev(a["mu"], device), _dev(a["q"], device), _dev(a["s"], device)
    R, T = _dev(a["R"], device), _dev(a["t"], device)
    mean2d, cov2d, depth = crc.project(n, mu, q, s, R, T, a["fx"], a["fy"], a["cx"], a["cy"])
    colors = crc.SH(n, _dev(a["cam"], device), mu, _dev(a["A"], device), _dev(a["kj"], device))
    alpha = _dev(a["alpha"], device)
    img, ids, ranges, fT, nc, keys = crc.rasterize_with_keys(n, depth, mean2d, cov2d, colors,
                                                             alpha, a["H"], a["W"])
    torch.cuda.synchronize()
    return dict(mean2d=_np(mean2d), cov2d=_np(cov2d), depth=_np(depth), colors=_np(colors),
                img=_np(img), ids=_np(ids), ranges=_np(ranges), final_T=_np(fT),
                n_contrib=_np(nc), keys=_np(keys).view(np.uint64), tensors=dict(
                    mean2d=mean2d, cov2d=cov2d, colors=colors, alpha=alpha, ids=ids,
                    ranges=ranges, final_T=fT, n_contrib=nc))


def _check_forward(got, want, images_bitwise=True):
    assert_bitwise(got["mean2d"], want["mean2d"], "mean2d")
    assert_bitwise(got["cov2d"], want["cov2d"], "cov2d")
    assert_bitwise(got["depth"], want["depth"], "depth")
    assert_bitwise(got["colors"], want["colors"], "colors")
    assert_bitwise(got["keys"], want["keys"], "sorted keys")
    assert_bitwise(got["ids"], want["ids"], "sorted_ids")
    assert_bitwise(got["ranges"], want["ranges"], "tile_ranges")
    assert_bitwise(got["n_contrib"], want["n_contrib"], "n_contrib")
    assert np.abs(got["img"] - want["img"]).max() <= 1e-5
    assert np.abs(got["final_T"] - want["final_T"]).max() <= 1e-5
    if images_bitwise:
        assert_bitwise(got["img"], want["img"], "img")
        assert_bitwise(got["final_T"], want["final_T"], "final_T")


SCENES = [
    ("c1", dict()),
    ("c2", dict(n=20_000, width=640, height=360)),
    ("c3", dict(n=20_000, width=480, height=270)),
    ("c4", dict(n=50_000, width=480, height=272)),
    ("c5", dict(n=30_000, width=400, height=224)),
]


@pytest.mark.parametrize("name,kw", SCENES, ids=[s[0] for s in SCENES])
def test_forward_parity_configs(crc, device, name, kw):
    print(f"[gpu] forward parity {name} {kw}", flush=True)
    sc = synthetic.config_scene(name, requires_grad=False, **kw)
    a = scene_arrays(sc)
    _check_forward(gpu_forward(crc, a, device), oracle_forward(a))


def test_forward_parity_bench_scene(crc, device):
    sc = synthetic.bench_scene(n=30_000, width=640, height=360, requires_grad=False)
    a = scene_arrays(sc)
    _check_forward(gpu_forward(crc, a, device), oracle_forward(a))


@pytest.mark.parametrize("binning", ["blocks", "sort"])
def test_forward_parity_600k_1080p(crc, device, monkeypatch, binning):
    """600k Gaussians at 1080p through both tile binnings: the two-level block
    binning, and the LSD tile sort (screens beyond its block histogram, or
    GSR_TILE_BINNING=sort), whose 20 id bits + 13 tile bits exceed one 32-bit
    word so keys and ids travel as separate words."""
    print(f"[gpu] forward parity, {binning} binning (600k Gaussians, 1920x1080)", flush=True)
    if binning == "sort":
        monkeypatch.setenv("GSR_TILE_BINNING", "sort")
    sc = synthetic.config_scene("c3", requires_grad=False, n=600_000, width=1920, height=1080)
    a = scene_arrays(sc)
    _check_forward(gpu_forward(crc, a, device), oracle_forward(a))


def test_4k_frame_properties(crc, device, monkeypatch):
    """1M Gaussians at 3840x2160 (32,400 tiles), beyond the oracle's seconds:
    size-independent properties instead.  Both tile binnings give the same
    keys, ids, ranges, n_contrib, image and final T bit for bit; every list is
    sorted by (depth bits, id) and holds only Gaussians whose tile rectangle
    covers the tile; the ranges tile [0, M); the backward is deterministic and
    finite."""
    print("[gpu] 4K frame properties (1M Gaussians, 3840x2160)", flush=True)
    sc = synthetic.config_scene("c3", requires_grad=False, n=1_000_000, width=3840, height=2160)
    a = scene_arrays(sc)
    blocks = gpu_forward(crc, a, device)
    monkeypatch.setenv("GSR_TILE_BINNING", "sort")
    srt = gpu_forward(crc, a, device)
    monkeypatch.delenv("GSR_TILE_BINNING")
    for k in ("keys", "ids", "ranges", "n_contrib", "img", "final_T"):
        assert_bitwise(blocks[k], srt[k], f"blocks vs sort: {k}")
    keys, ids, rng = blocks["keys"], blocks["ids"].astype(np.int64), blocks["ranges"]
    M = ids.size
    assert M > 10_000_000
    tiles = (keys >> np.uint64(32)).astype(np.int64)
    assert np.all(keys[1:] >= keys[:-1])
    same = (keys[1:] == keys[:-1])
    assert np.all(ids[1:][same] > ids[:-1][same]), "equal keys keep the Gaussian order"
    nz = rng[:, 1] > rng[:, 0]
    assert rng[nz, 0].min() == 0 and rng[nz, 1].max() == M
    assert np.array_equal(np.sort(rng[nz, 0]), rng[nz, 0]) and np.all(rng[nz][1:, 0] == rng[nz][:-1, 1])
    # the tile of each pair lies in its Gaussian's tile rectangle
    _, rect = orc.bin_count(blocks["mean2d"], blocks["cov2d"], a["H"], a["W"])
    x0, x1, y0, y1 = (rect[:, k][ids] for k in range(4))
    tx_n = (a["W"] + 15) // 16
    tx, ty = tiles % tx_n, tiles // tx_n
    assert np.all((tx >= x0) & (tx < x1) & (ty >= y0) & (ty < y1))
    t, n = blocks["tensors"], a["mu"].shape[0]
    G = synthetic.grad_image(a["H"], a["W"], seed=5).to(device)
    args = (t["mean2d"], t["cov2d"], t["colors"], t["alpha"], t["ids"], t["ranges"], t["final_T"],
            t["n_contrib"], n, a["H"], a["W"])
    r1 = [_np(x) for x in crc.backwards_rasterization(G, *args)]
    r2 = [_np(x) for x in crc.backwards_rasterization(G, *args)]
    for x, y, nm in zip(r1, r2, ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert np.isfinite(x).all(), nm
        assert_bitwise(x, y, nm)


@pytest.mark.parametrize("name,kw", [("c3", dict(n=20_000, width=480, height=270)),
                                     ("c5", dict(n=30_000, width=400, height=224))],
                         ids=["c3", "c5"])
def test_forward_parity_tile_sort(crc, device, monkeypatch, name, kw):
    """The LSD tile sort (packed words) that serves screens with more 8x8-tile
    blocks than the block binning's histogram holds."""
    monkeypatch.setenv("GSR_TILE_BINNING", "sort")
    a = scene_arrays(synthetic.config_scene(name, requires_grad=False, **kw))
    _check_forward(gpu_forward(crc, a, device), oracle_forward(a))


@pytest.mark.parametrize("H,W", [(16, 16), (17, 33), (1, 1), (100, 7), (240, 321)])
def test_forward_parity_odd_screens(crc, device, H, W):
    sc = synthetic.config_scene("c1", requires_grad=False, n=3000, width=W, height=H)
    a = scene_arrays(sc)
    _check_forward(gpu_forward(crc, a, device), oracle_forward(a))


def test_projection_wide_ranges_bitwise(crc, device):
    """Random poses, log-scales over [-12, 4] (exp over a wide range), culled points."""
    rng = np.random.default_rng(5)
    n = 200_000
    mu = np.c_[rng.uniform(-3, 3, (n, 2)), rng.uniform(-1, 8, n)].astype(np.float32)
    q = rng.normal(size=(n, 4)).astype(np.float32)
    q[::97] = 0.0
    s = rng.uniform(-12, 4, (n, 3)).astype(np.float32)
    ang = rng.normal(size=4)
    w, x, y, z = ang / np.linalg.norm(ang)
    R = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                  [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                  [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]], np.float32)
    t = np.array([0.1, -0.2, 0.5], np.float32)
    want = orc.project(mu, q, s, R, t, 811.0, 799.5, 640.0, 360.0)
    got = crc.project(n, _dev(mu, device), _dev(q, device), _dev(s, device), _dev(R, device),
                      _dev(t, device), 811.0, 799.5, 640.0, 360.0)
    for g, w_, nm in zip(got, want, ("mean2d", "cov2d", "depth")):
        assert_bitwise(_np(g), w_, nm)


def test_sh_bitwise(crc, device):
    rng = np.random.default_rng(6)
    n = 100_000
    mu = rng.normal(size=(n, 3)).astype(np.float32) * 3
    A = rng.uniform(-2, 2, (n, 3)).astype(np.float32)
    kj = rng.normal(0, 0.3, (n, 15, 3)).astype(np.float32)
    cam = np.array([0.3, -0.1, -2.0], np.float32)
    want = orc.sh(cam, mu, A, kj)
    got = crc.SH(n, _dev(cam, device), _dev(mu, device), _dev(A, device), _dev(kj, device))
    assert_bitwise(_np(got), want, "colors")


def test_unaligned_views_are_accepted(crc, device):
    """Contiguous views that start 4 bytes into their storage (the reference
    accepts them): quaternions and SH coefficients are realigned internally."""
    rng = np.random.default_rng(11)
    n = 1000
    mu = rng.normal(size=(n, 3)).astype(np.float32)
    mu[:, 2] += 5.0
    q = rng.normal(size=(n, 4)).astype(np.float32)
    s = rng.uniform(-4, -2, (n, 3)).astype(np.float32)
    R, t = np.eye(3, dtype=np.float32), np.zeros(3, np.float32)
    qbig = _dev(np.r_[np.zeros(1, np.float32), q.ravel()], device)[1:].view(n, 4)
    assert qbig.data_ptr() % 16 == 4
    got = crc.project(n, _dev(mu, device), qbig, _dev(s, device), _dev(R, device), _dev(t, device),
                      300.0, 300.0, 64.0, 48.0)
    want = orc.project(mu, q, s, R, t, 300.0, 300.0, 64.0, 48.0)
    for g, w_, nm in zip(got, want, ("mean2d", "cov2d", "depth")):
        assert_bitwise(_np(g), w_, nm)
    A = rng.uniform(0, 1, (n, 3)).astype(np.float32)
    kj = rng.normal(0, 0.2, (n, 15, 3)).astype(np.float32)
    cam = np.array([0.1, 0.2, -1.0], np.float32)
    kbig = _dev(np.r_[np.zeros(1, np.float32), kj.ravel()], device)[1:].view(n, 15, 3)
    got = crc.SH(n, _dev(cam, device), _dev(mu, device), _dev(A, device), kbig)
    assert_bitwise(_np(got), orc.sh(cam, mu, A, kj), "colors")


def test_glue_radii_and_camera_position(crc, device):
    """The glue's one-kernel screen radii equal the torch formula of the
    reference's rasterize.py:49-53 bit for bit (NaN kept, clamps hit), and its
    camera position is -R^T t to fp32 rounding."""
    rng = np.random.default_rng(12)
    n = 50_000
    cov = np.c_[rng.uniform(-0.5, 40, n), rng.normal(0, 5, n), rng.uniform(-0.5, 40, n)].astype(np.float32)
    cov[:5] = [[0.0, 0.0, 0.0], [np.nan, 1.0, 2.0], [-3.0, 0.0, -3.0], [1e-3, 0.0, 1e-3], [np.inf, 0.0, 1.0]]
    c = _dev(cov, device)
    a, b, cc = c[:, 0], c[:, 1], c[:, 2]
    mid = 0.5 * (a + cc)
    radius = mid + torch.sqrt(torch.clamp((0.5 * (a - cc)) ** 2 + b * b, min=0.1))
    want = 3.0 * torch.sqrt(torch.clamp(radius, min=0.0))
    got = crc.screen_radii(c)
    assert_bitwise(_np(got), _np(want), "radii")
    ang = rng.normal(size=4)
    w, x, y, z = ang / np.linalg.norm(ang)
    R = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                  [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                  [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]], np.float32)
    tt = np.array([0.3, -1.2, 2.5], np.float32)
    cam = _np(crc.camera_position(_dev(R, device), _dev(tt, device)))
    ref = -(R.astype(np.float64).T @ tt.astype(np.float64))
    assert np.abs(cam - ref).max() <= 4e-7 * np.abs(ref).max()


def test_empty_frames(crc, device):
    f = lambda *s: torch.zeros(*s, device=device)
    img, ids, ranges, fT, nc = crc.rasterize(0, f(0), f(0, 2), f(0, 3), f(0, 3), f(0), 40, 50)
    assert img.shape == (40, 50, 3) and float(img.abs().sum()) == 0
    assert ids.numel() == 0 and ranges.shape == (12, 2) and int(ranges.abs().sum()) == 0
    assert bool((fT == 1).all()) and int(nc.abs().sum()) == 0
    # every Gaussian culled (zero covariance -> det <= 0 -> no tiles)
    n = 10
    img, ids, ranges, fT, nc = crc.rasterize(n, f(n) + 1, f(n, 2) + 5, f(n, 3), f(n, 3),
                                             f(n) + 0.5, 32, 32)
    assert ids.numel() == 0 and bool((fT == 1).all()) and float(img.abs().sum()) == 0
    assert ranges.dtype == torch.int32 and nc.dtype == torch.int32


def test_input_checks(crc, device):
    n = 4
    good = lambda *s: torch.zeros(*s, device=device)
    with pytest.raises(RuntimeError, match="mean_2d must have shape"):
        crc.rasterize(n, good(n), good(n, 3), good(n, 3), good(n, 3), good(n), 16, 16)
    with pytest.raises(RuntimeError, match="must be contiguous"):
        crc.rasterize(n, good(n), good(2, n).t(), good(n, 3), good(n, 3), good(n), 16, 16)
    with pytest.raises(RuntimeError, match="must be FP32"):
        crc.rasterize(n, good(n), good(n, 2).double(), good(n, 3), good(n, 3), good(n), 16, 16)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        crc.rasterize(n, good(n).cpu(), good(n, 2), good(n, 3), good(n, 3), good(n), 16, 16)


def _backward_case(crc, device, a, seed=3, corrupt=False):
    fw = gpu_forward(crc, a, device)
    want = oracle_forward(a)
    assert_bitwise(fw["n_contrib"], want["n_contrib"], "n_contrib")
    H, W = a["H"], a["W"]
    G = synthetic.grad_image(H, W, seed=seed).numpy()
    t = fw["tensors"]
    ids = t["ids"]
    ids_np = want["ids"].copy()
    if corrupt and ids_np.size > 10:
        pos = np.random.default_rng(0).choice(ids_np.size, 8, replace=False)
        ids_np[pos[:4]] = -1
        ids_np[pos[4:]] = a["mu"].shape[0] + 5
        ids = _dev(ids_np, device, torch.int32)
    n = a["mu"].shape[0]
    dm, dc, dcol, dal = crc.backwards_rasterization(
        _dev(G, device), t["mean2d"], t["cov2d"], t["colors"], t["alpha"], ids, t["ranges"],
        t["final_T"], t["n_contrib"], n, H, W)
    torch.cuda.synchronize()
    ref = orc.blend_bwd(G, want["mean2d"], want["cov2d"], want["colors"], a["alpha"], ids_np,
                        want["ranges"], want["final_T"], want["n_contrib"], H, W, with_abs=True)
    for got_t, r, ab, nm in zip((dm, dc, dcol, dal), ref[:4], ref[4:], ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert_grad_close(_np(got_t), r, ab, nm)
    assert dal.shape == (n, 1)
    return fw, want, G, (dm, dc, dcol, dal)


@pytest.mark.parametrize("name,kw", [("c1", dict()), ("c2", dict(n=20_000, width=640, height=360)),
                                     ("c3", dict(n=20_000, width=480, height=270)),
                                     ("c4", dict(n=50_000, width=480, height=272)),
                                     ("c5", dict(n=20_000, width=320, height=192)),
                                     ("c3_1080p", dict(n=60_000, width=1920, height=1080))],
                         ids=["c1", "c2", "c3", "c4", "c5", "c3_1080p"])
def test_rasterize_backward_parity(crc, device, name, kw):
    """c3_1080p: 8160 tiles, more than fit on the device at once, so the
    backward runs its 64-entry-batch kernel."""
    print(f"[gpu] backward parity {name} {kw}", flush=True)
    a = scene_arrays(synthetic.config_scene(name.split("_")[0], requires_grad=False, **kw))
    _backward_case(crc, device, a)


def test_rasterize_backward_parity_large_splats(crc, device):
    """Gaussians covering hundreds of tiles each (c3's cloud with log-scales
    raised by 3): more than 256 gradient slots per Gaussian, so each row of
    the gradient reduce walks several flag groups; against the oracle as every
    backward case."""
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=2000, width=640,
                                            height=368))
    a["s"] = (a["s"] + 3.0).astype(np.float32)
    fw, want, G, _ = _backward_case(crc, device, a)
    assert fw["ids"].size > 256 * a["mu"].shape[0]


def test_rasterize_backward_split_tiles(crc, device, monkeypatch):
    """The backward runs its longest tiles as two work items: a back part from
    the final transmittance, and a front part that walks the back part's
    entries with the pixel state only before its own.  On c4's clustered
    cloud (long lists; the largest tiles split) the gradients are within the
    oracle bar and bit for bit the unsplit backward's (GSR_BWD_SPLIT=0), also
    with ids the forward did not produce in the lists."""
    a = scene_arrays(synthetic.config_scene("c4", requires_grad=False, n=50_000, width=480,
                                            height=272))
    fw, want, G, split = _backward_case(crc, device, a)
    t, n = fw["tensors"], a["mu"].shape[0]
    monkeypatch.setenv("GSR_BWD_SPLIT", "0")
    whole = crc.backwards_rasterization(
        _dev(G, device), t["mean2d"], t["cov2d"], t["colors"], t["alpha"], t["ids"], t["ranges"],
        t["final_T"], t["n_contrib"], n, a["H"], a["W"])
    for x, y, nm in zip(split, whole, ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert_bitwise(_np(x), _np(y), f"split vs whole: {nm}")
    # ids the forward did not produce (skipped entries) on both paths
    ids = _np(t["ids"]).copy()
    pos = np.random.default_rng(1).choice(ids.size, 64, replace=False)
    ids[pos[:32]] = -1
    ids[pos[32:]] = n + 7
    bad = _dev(ids, device, torch.int32)
    args = (_dev(G, device), t["mean2d"], t["cov2d"], t["colors"], t["alpha"], bad, t["ranges"],
            t["final_T"], t["n_contrib"], n, a["H"], a["W"])
    whole = crc.backwards_rasterization(*args)
    monkeypatch.setenv("GSR_BWD_SPLIT", "1")
    split = crc.backwards_rasterization(*args)
    for x, y, nm in zip(split, whole, ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert_bitwise(_np(x), _np(y), f"split vs whole, corrupt ids: {nm}")


def test_rasterize_backward_strided_gradient_views(crc, device):
    """backwards_rasterization_strided reads dL/dimage views in place: a
    broadcast (image.sum()'s gradient, strides 0), a transposed image and a
    channel slice, each bit for bit the contiguous op on .contiguous()."""
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=20_000, width=480,
                                            height=270))
    fw = gpu_forward(crc, a, device)
    t, n, H, W = fw["tensors"], a["mu"].shape[0], a["H"], a["W"]
    G = synthetic.grad_image(H, W, seed=4).to(device)
    views = {
        "broadcast": torch.full((1, 1, 1), 1.7, device=device).expand(H, W, 3),
        "transposed": G.transpose(0, 1).contiguous().transpose(0, 1),
        "channel_slice": torch.cat([G, G[..., :1]], dim=2)[..., :3],
    }
    for name, g in views.items():
        assert not g.is_contiguous(), name
        args = (t["mean2d"], t["cov2d"], t["colors"], t["alpha"], t["ids"], t["ranges"],
                t["final_T"], t["n_contrib"], n, H, W)
        want = crc.backwards_rasterization(g.contiguous(), *args)
        got = crc.backwards_rasterization_strided(g, *args)
        for x, y, nm in zip(got, want, ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
            assert_bitwise(_np(x), _np(y), f"{name}: {nm}")
    with pytest.raises(RuntimeError, match="contiguous"):
        crc.backwards_rasterization(views["transposed"], *args)
    with pytest.raises(RuntimeError, match="shape"):
        crc.backwards_rasterization_strided(G.reshape(W, H, 3), *args)


def test_rasterize_backward_skips_corrupt_ids(crc, device):
    a = scene_arrays(synthetic.config_scene("c1", requires_grad=False, n=2000, width=64, height=48))
    _backward_case(crc, device, a, corrupt=True)


def test_rasterize_backward_inputs_off_the_rectangles(crc, device):
    """Backward inputs whose (Gaussian, tile) pairs do not all lie in the tile
    rectangles of mean2d/cov2d (the reference takes sorted ids and ranges as
    given): such pairs take the direct path and must still match."""
    a = scene_arrays(synthetic.config_scene("c1", requires_grad=False, n=3000, width=96, height=64))
    fw = gpu_forward(crc, a, device)
    want = oracle_forward(a)
    H, W = a["H"], a["W"]
    G = synthetic.grad_image(H, W, seed=5).numpy()
    t = fw["tensors"]
    cov = (want["cov2d"] * np.float32(0.25)).astype(np.float32)  # smaller rectangles
    n = a["mu"].shape[0]
    got = crc.backwards_rasterization(_dev(G, device), t["mean2d"], _dev(cov, device), t["colors"],
                                      t["alpha"], t["ids"], t["ranges"], t["final_T"],
                                      t["n_contrib"], n, H, W)
    torch.cuda.synchronize()
    ref = orc.blend_bwd(G, want["mean2d"], cov, want["colors"], a["alpha"], want["ids"],
                        want["ranges"], want["final_T"], want["n_contrib"], H, W, with_abs=True)
    for got_t, r, ab, nm in zip(got, ref[:4], ref[4:], ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert_grad_close(_np(got_t), r, ab, nm)


def _threshold_scene(seed=17, H=48, W=64, crafted=600, others=500):
    """2D inputs whose skips sit on the edges: `crafted` Gaussians each put one
    pixel's alpha within a few ulp of 1/255 (variance 0.25-0.35 px^2, mean
    0.2-0.45 px from the pixel, so every other pixel's alpha is below 0.9/255),
    and `others` of 1-6 px with opacities in (0, 1), at and above the 0.99
    clamp, zero and negative."""
    rng = np.random.default_rng(seed)
    f32 = np.float32
    px = rng.integers(2, W - 2, crafted).astype(f32)
    py = rng.integers(2, H - 2, crafted).astype(f32)
    mx = (px - rng.uniform(0.2, 0.45, crafted)).astype(f32)
    my = (py - rng.uniform(0.2, 0.45, crafted)).astype(f32)
    var = rng.uniform(0.25, 0.35, crafted).astype(f32)
    # the blend's power at (px, py) in fp32 (rasterize.cu:249-251); conic.y = -0
    inv = (f32(1.0) / (var * var)).astype(f32)
    cn = (var * inv).astype(f32)
    dx, dy = (px - mx).astype(f32), (py - my).astype(f32)
    power = (f32(-0.5) * ((cn * dx) * dx + (cn * dy) * dy)).astype(f32)
    G = orc.expf_array(power).astype(f32)
    o = (f32(1.0 / 255.0) / G).astype(f32)
    for i, k in enumerate(rng.integers(-4, 5, crafted)):
        for _ in range(abs(int(k))):
            o[i] = np.nextafter(o[i], f32(np.inf) if k > 0 else f32(0.0))
    mean = [np.stack([mx, my], 1)]
    cov = [np.stack([var, np.zeros_like(var), var], 1)]
    opac = [o]
    sig = rng.uniform(1.0, 6.0, (others, 2))
    rho = rng.uniform(-0.8, 0.8, others)
    mean.append(np.stack([rng.uniform(-4, W + 4, others), rng.uniform(-4, H + 4, others)], 1))
    cov.append(np.stack([sig[:, 0] ** 2, rho * sig[:, 0] * sig[:, 1], sig[:, 1] ** 2], 1))
    oth = rng.uniform(0.0, 1.0, others)
    pick = rng.integers(0, 8, others)
    oth = np.where(pick == 0, rng.choice([0.99, 0.995, 1.0, 3.0], others), oth)
    oth = np.where(pick == 1, rng.choice([0.0, -0.3, 0.98999994], others), oth)
    opac.append(oth)
    mean2d = np.concatenate(mean).astype(f32)
    cov2d = np.concatenate(cov).astype(f32)
    alpha = np.concatenate(opac).astype(f32).reshape(-1, 1)
    n = alpha.shape[0]
    depth = rng.uniform(0.5, 20.0, n).astype(f32)
    colors = rng.uniform(0.0, 1.0, (n, 3)).astype(f32)
    return dict(H=H, W=W, mean2d=mean2d, cov2d=cov2d, alpha=alpha, depth=depth, colors=colors)


def test_forward_parity_nonfinite_colours(crc, device):
    """Entries with an infinite colour channel take the forward's select path
    (a skipped entry must not add inf * 0); images, final T and n_contrib
    equal the oracle's bit for bit, infinities included."""
    s = _threshold_scene(seed=23)
    n = s["alpha"].shape[0]
    rng = np.random.default_rng(5)
    pick = rng.choice(np.arange(600, n), 12, replace=False)
    s["colors"][pick, rng.integers(0, 3, 12)] = np.float32(np.inf)
    H, W = s["H"], s["W"]
    t = {k: _dev(s[k], device) for k in ("depth", "mean2d", "cov2d", "colors", "alpha")}
    img, ids, ranges, fT, nc, _ = crc.rasterize_with_keys(n, t["depth"], t["mean2d"], t["cov2d"],
                                                          t["colors"], t["alpha"], H, W)
    w_img, w_ids, w_rng, w_fT, w_nc, _ = orc.rasterize(s["depth"], s["mean2d"], s["cov2d"],
                                                       s["colors"], s["alpha"], H, W)
    assert np.isinf(w_img).any()
    assert_bitwise(_np(ids), w_ids, "sorted_ids")
    assert_bitwise(_np(nc), w_nc, "n_contrib")
    assert_bitwise(_np(img), w_img, "img")
    assert_bitwise(_np(fT), w_fT, "final_T")


def test_rasterize_backward_alpha_at_the_thresholds(crc, device):
    """The backward's skips (power > 0, alpha < 1/255, the 0.99 clamp) must be
    the forward's bit for bit, also where alpha is within a few ulp of 1/255:
    forward n_contrib exact, gradients within the fp32 bar."""
    s = _threshold_scene()
    H, W, n = s["H"], s["W"], s["alpha"].shape[0]
    t = {k: _dev(s[k], device) for k in ("depth", "mean2d", "cov2d", "colors", "alpha")}
    img, ids, ranges, fT, nc, _ = crc.rasterize_with_keys(n, t["depth"], t["mean2d"], t["cov2d"],
                                                          t["colors"], t["alpha"], H, W)
    want = orc.rasterize(s["depth"], s["mean2d"], s["cov2d"], s["colors"], s["alpha"], H, W)
    w_img, w_ids, w_rng, w_fT, w_nc, _ = want
    assert_bitwise(_np(ids), w_ids, "sorted_ids")
    assert_bitwise(_np(nc), w_nc, "n_contrib")
    assert np.abs(_np(img) - w_img).max() <= 1e-5
    G = synthetic.grad_image(H, W, seed=4).numpy()
    got = crc.backwards_rasterization(_dev(G, device), t["mean2d"], t["cov2d"], t["colors"],
                                      t["alpha"], ids, ranges, fT, nc, n, H, W)
    torch.cuda.synchronize()
    ref = orc.blend_bwd(G, s["mean2d"], s["cov2d"], s["colors"], s["alpha"], w_ids, w_rng, w_fT,
                        w_nc, H, W, with_abs=True)
    for got_t, r, ab, nm in zip(got, ref[:4], ref[4:], ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert_grad_close(_np(got_t), r, ab, nm)
    # the crafted Gaussians' single-pixel contributions decide d_alpha on their own
    crafted = 600
    live = np.abs(ref[3][:crafted]).ravel() > 0
    assert live.any() and (~live).any()
    assert np.array_equal(np.abs(_np(got[3])[:crafted]).ravel() > 0, live)


def test_rasterize_backward_is_deterministic(crc, device):
    """Each Gaussian's gradient is a fixed-order sum of its per-tile slots."""
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=30_000, width=480, height=270))
    fw = gpu_forward(crc, a, device)
    t = fw["tensors"]
    G = _dev(synthetic.grad_image(a["H"], a["W"], seed=2).numpy(), device)
    n = a["mu"].shape[0]
    args = (G, t["mean2d"], t["cov2d"], t["colors"], t["alpha"], t["ids"], t["ranges"],
            t["final_T"], t["n_contrib"], n, a["H"], a["W"])
    r1 = [_np(x) for x in crc.backwards_rasterization(*args)]
    r2 = [_np(x) for x in crc.backwards_rasterization(*args)]
    for x, y, nm in zip(r1, r2, ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert_bitwise(x, y, nm)


def test_sh_and_projection_backward_parity(crc, device):
    rng = np.random.default_rng(9)
    n = 50_000
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=n))
    cg = rng.normal(size=(n, 3)).astype(np.float32)
    want = orc.sh_bwd(cg, a["mu"], a["A"], a["kj"], a["cam"])
    got = crc.backwards_SH(_dev(cg, device), _dev(a["mu"], device), _dev(a["A"], device),
                           _dev(a["kj"], device), _dev(a["cam"], device))
    for g, w, nm in zip(got, want, ("d_albedo", "d_k_j", "d_mu_sh")):
        assert_bitwise(_np(g), w, nm)
    dm = rng.normal(size=(n, 2)).astype(np.float32)
    dc = rng.normal(size=(n, 3)).astype(np.float32)
    want = orc.project_bwd(dm, dc, a["mu"], a["q"], a["s"], a["R"], a["t"], a["fx"], a["fy"],
                           a["cx"], a["cy"])
    got = crc.backwards_projection(_dev(dm, device), _dev(dc, device), _dev(a["mu"], device),
                                   _dev(a["q"], device), _dev(a["s"], device), _dev(a["R"], device),
                                   _dev(a["t"], device), a["fx"], a["fy"], a["cx"], a["cy"])
    for g, w, nm in zip(got, want, ("d_mu", "d_q", "d_s")):
        assert_bitwise(_np(g), w, nm)


@pytest.mark.parametrize("n", [50_003, 64, 1])
def test_project_sh_matches_the_separate_ops(crc, device, n):
    """The glue's fused forward head: bit for bit camera_position, project,
    screen_radii and SH (and the oracle's projection and SH), culled points and
    a partial last work-group included."""
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=max(n, 2)))
    mu, q, s = (_dev(a[k][:n], device) for k in ("mu", "q", "s"))
    mu[::7, 2] = -1.0  # behind the camera: culled
    A, kj = _dev(a["A"][:n], device), _dev(a["kj"][:n], device)
    R, T = _dev(a["R"], device), _dev(a["t"], device)
    cam0 = crc.camera_position(R, T)
    sep = crc.project(n, mu, q, s, R, T, a["fx"], a["fy"], a["cx"], a["cy"])
    sep = (*sep, crc.screen_radii(sep[1]), crc.SH(n, cam0, mu, A, kj), cam0)
    got = crc.project_sh(n, mu, q, s, R, T, a["fx"], a["fy"], a["cx"], a["cy"], A, kj)
    for g, w, nm in zip(got, sep, ("mean2d", "cov2d", "depth", "radii", "colors", "cam")):
        assert_bitwise(_np(g), _np(w), nm)
    want = orc.project(_np(mu), _np(q), _np(s), a["R"], a["t"], a["fx"], a["fy"], a["cx"], a["cy"])
    for g, w, nm in zip(got[:3], want, ("mean2d", "cov2d", "depth")):
        assert_bitwise(_np(g), w, nm)
    assert_bitwise(_np(got[4]), orc.sh(_np(got[5]), _np(mu), _np(A), _np(kj)), "colors")


def test_project_sh_opacity_is_torch_sigmoid(crc, device):
    """The fused head's opacity from logits equals t.sigmoid bit for bit, over
    ±100, tiny and huge values, ±inf and NaN; the fused tail's logit gradient
    equals torch's sigmoid backward bit for bit."""
    rng = np.random.default_rng(23)
    n = 70_001
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=n))
    lg = np.r_[rng.uniform(-100, 100, n - 9),
               [0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, np.inf, -np.inf, np.nan]].astype(np.float32)
    logits = _dev(lg.reshape(n, 1), device)
    mu, q, s = (_dev(a[k], device) for k in ("mu", "q", "s"))
    A, kj = _dev(a["A"], device), _dev(a["kj"], device)
    R, T = _dev(a["R"], device), _dev(a["t"], device)
    out = crc.project_sh(n, mu, q, s, R, T, a["fx"], a["fy"], a["cx"], a["cy"], A, kj, logits)
    op = out[6]
    assert op.shape == logits.shape
    assert_bitwise(_np(op), _np(torch.sigmoid(logits)), "opacity")
    dop = _dev(rng.normal(size=(n, 1)), device)
    z = lambda *sh: torch.zeros(*sh, device=device)
    got = crc.backwards_project_sh(z(n, 2), z(n, 3), z(n, 3), mu, q, s, R, T, a["fx"], a["fy"],
                                   A, kj, out[5], dop, op)
    assert got[5].shape == op.shape
    assert_bitwise(_np(got[5]), _np(torch.ops.aten.sigmoid_backward(dop, op)), "d logits")
    assert got[5].numel() == n and crc.backwards_project_sh(
        z(n, 2), z(n, 3), z(n, 3), mu, q, s, R, T, a["fx"], a["fy"], A, kj, out[5])[5].numel() == 0


def test_glue_logits_path_equals_sigmoid_then_rasterize(device):
    """rasterize() (opacity logits, sigmoid fused) against t.sigmoid +
    RasterizeFunction: the image and every parameter gradient bit for bit."""
    import importlib
    glue = importlib.import_module("gaussian_splatting.rasterizer.rasterize")
    sc = synthetic.config_scene("c3", device=device, n=20_000, width=480, height=270)
    g, v = sc.gaussians, sc.view
    names = ("mu", "q", "s", "alpha", "A", "k_j")

    def run(fused):
        for nm in names:
            getattr(g, nm).grad = None
        if fused:
            img = glue.rasterize(g, v)
        else:
            img = glue.RasterizeFunction.apply(g.mu, g.q, g.s, torch.sigmoid(g.alpha), g.A, g.k_j,
                                               v["R"], v["T"], v["fx"], v["fy"], v["cx"],
                                               v["cy"], v["height"], v["width"])
        (img * torch.linspace(0.5, 1.5, img.numel(), device=device).view_as(img)).sum().backward()
        return img.detach().clone(), [getattr(g, nm).grad.clone() for nm in names]

    i1, g1 = run(True)
    i0, g0 = run(False)
    assert_bitwise(_np(i1), _np(i0), "image")
    for a_, b_, nm in zip(g1, g0, names):
        assert_bitwise(_np(a_), _np(b_), f"d {nm}")


def test_project_sh_without_gaussians_gives_the_camera(crc, device):
    a = scene_arrays(synthetic.config_scene("c1", requires_grad=False))
    R, T = _dev(a["R"], device), _dev(a["t"], device)
    z3 = torch.zeros(0, 3, device=device)
    out = crc.project_sh(0, z3, torch.zeros(0, 4, device=device), z3, R, T, a["fx"], a["fy"],
                         a["cx"], a["cy"], z3, torch.zeros(0, 15, 3, device=device))
    assert [tuple(x.shape) for x in out[:5]] == [(0, 2), (0, 3), (0,), (0,), (0, 3)]
    assert_bitwise(_np(out[5]), _np(crc.camera_position(R, T)), "cam")


@pytest.mark.parametrize("n", [50_003, 1])
def test_backwards_project_sh_matches_the_separate_ops(crc, device, n):
    """The glue's fused backward tail: bit for bit backwards_SH,
    backwards_projection and mu_grad + mu_sh_grad (and the oracle's)."""
    rng = np.random.default_rng(21)
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=max(n, 2)))
    mu, q, s = (_dev(a[k][:n], device) for k in ("mu", "q", "s"))
    mu[::5, 2] = -1.0
    A, kj = _dev(a["A"][:n], device), _dev(a["kj"][:n], device)
    R, T, cam = _dev(a["R"], device), _dev(a["t"], device), _dev(a["cam"], device)
    dm = _dev(rng.normal(size=(n, 2)), device)
    dc = _dev(rng.normal(size=(n, 3)), device)
    cg = _dev(rng.normal(size=(n, 3)), device)
    dA, dkj, dmu_sh = crc.backwards_SH(cg, mu, A, kj, cam)
    dmu_p, dq, ds = crc.backwards_projection(dm, dc, mu, q, s, R, T, a["fx"], a["fy"], a["cx"],
                                             a["cy"])
    got = crc.backwards_project_sh(dm, dc, cg, mu, q, s, R, T, a["fx"], a["fy"], A, kj, cam)
    for g, w, nm in zip(got, (dmu_p + dmu_sh, dq, ds, dA, dkj),
                        ("d_mu", "d_q", "d_s", "d_albedo", "d_k_j")):
        assert_bitwise(_np(g), _np(w), nm)
    w_sh = orc.sh_bwd(_np(cg), _np(mu), _np(A), _np(kj), a["cam"])
    w_p = orc.project_bwd(_np(dm), _np(dc), _np(mu), _np(q), _np(s), a["R"], a["t"], a["fx"],
                          a["fy"], a["cx"], a["cy"])
    assert_bitwise(_np(got[0]), (w_p[0] + w_sh[2]).astype(np.float32), "d_mu (oracle)")
    for g, w, nm in zip(got[1:], (w_p[1], w_p[2], w_sh[0], w_sh[1]),
                        ("d_q", "d_s", "d_albedo", "d_k_j")):
        assert_bitwise(_np(g), w, nm + " (oracle)")


def test_forward_is_deterministic(crc, device):
    a = scene_arrays(synthetic.config_scene("c2", requires_grad=False, n=40_000))
    r1 = gpu_forward(crc, a, device)
    r2 = gpu_forward(crc, a, device)
    for k in ("keys", "ids", "ranges", "n_contrib", "img", "final_T"):
        assert_bitwise(r1[k], r2[k], k)
