"""Seeded synthetic scenes for tests and benchmarks.

* ``bench_scene`` — the reference's benchmark cloud and camera
  (scripts/bench.py:30-63): z ~ U(2,6), x ~ U(-.35,.35) z, y ~ U(-.25,.25) z,
  identity quaternions, log-scale -3, opacity logit 0, SH all zero; identity
  pose, fx = fy = W, cx = W/2, cy = H/2.  Same torch CPU generator calls in the
  same order, so the same seed gives the same cloud.
* ``config_scene`` — the configurations c1..c5 of the rasterizer baseline:
  identity pose, pinhole with a 60 degree horizontal field of view
  (fx = fy = (W/2)/tan 30deg), means x, y ~ U[-1,1], z ~ U[2,6], log-scales
  N(-4, 0.5), quaternions normalize(N(0,1)^4), opacity logits N(0,1),
  c1: SH degree 0 (k_j = 0, albedo = (rgb - 0.5)/C0, rgb ~ U[0,1]);
  c2/c3: albedo ~ U[0,1], k_j ~ N(0, 0.1);
  c4: as c3 with 80% of means at z ~ U[3, 3.5], x, y uniform inside the frustum;
  c5: as c3 with one random axis log-scale N(-2, 0.5), others N(-5, 0.5),
      opacity logits N(-1, 1).
All tensors are generated on the CPU and moved to ``device`` afterwards, so the
GPU path and the CPU oracle consume identical bits.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch as t

from gaussian_splatting.scene.gaussian import gaussian

SH_C0 = 0.28209479177387814

CONFIGS = {
    "c1": dict(n=10_000, width=256, height=256, sh="dc"),
    "c2": dict(n=100_000, width=1280, height=720, sh="full"),
    "c3": dict(n=100_000, width=1920, height=1080, sh="full"),
    "c4": dict(n=1_000_000, width=1920, height=1080, sh="full", clustered=True),
    "c5": dict(n=5_000_000, width=3840, height=2160, sh="full", anisotropic=True),
}


@dataclass
class Scene:
    gaussians: gaussian
    view: dict
    name: str

    @property
    def n(self) -> int:
        return self.gaussians.mu.shape[0]


def _finish(g: gaussian, device, requires_grad: bool) -> gaussian:
    for name in ("mu", "q", "s", "alpha", "A", "k_j"):
        v = getattr(g, name).to(device=device, dtype=t.float32).contiguous()
        if requires_grad:
            v.requires_grad_(True)
        setattr(g, name, v)
    return g


def bench_view(width: int, height: int, device) -> dict:
    return {
        "R": t.eye(3, device=device, dtype=t.float32),
        "T": t.zeros(3, device=device, dtype=t.float32),
        "fx": float(width),
        "fy": float(width),
        "cx": width * 0.5,
        "cy": height * 0.5,
        "height": height,
        "width": width,
    }


def bench_scene(n: int = 100_000, width: int = 1920, height: int = 1080, device="cpu",
                seed: int = 0, requires_grad: bool = True) -> Scene:
    gen = t.Generator(device="cpu")
    gen.manual_seed(seed)
    z = t.empty(n, 1).uniform_(2.0, 6.0, generator=gen)
    x = t.empty(n, 1).uniform_(-0.35, 0.35, generator=gen) * z
    y = t.empty(n, 1).uniform_(-0.25, 0.25, generator=gen) * z
    g = gaussian(n)
    g.mu = t.cat((x, y, z), dim=1)
    g.q = t.zeros(n, 4)
    g.q[:, 0] = 1.0
    g.s = t.full((n, 3), -3.0)
    g.alpha = t.zeros(n, 1)
    g.A = t.zeros(n, 3)
    g.k_j = t.zeros(n, 15, 3)
    return Scene(_finish(g, device, requires_grad), bench_view(width, height, device),
                 f"bench_{width}x{height}")


def fov_view(width: int, height: int, device, fov_deg: float = 60.0) -> dict:
    f = (width / 2.0) / math.tan(math.radians(fov_deg) / 2.0)
    return {
        "R": t.eye(3, device=device, dtype=t.float32),
        "T": t.zeros(3, device=device, dtype=t.float32),
        "fx": f,
        "fy": f,
        "cx": width * 0.5,
        "cy": height * 0.5,
        "height": height,
        "width": width,
    }


def config_scene(name: str, device="cpu", seed: int = 0, requires_grad: bool = True,
                 n: int | None = None, width: int | None = None,
                 height: int | None = None) -> Scene:
    """BASELINE config ``name`` (c1..c5); n/width/height override the sizes."""
    cfg = dict(CONFIGS[name])
    n = n if n is not None else cfg["n"]
    width = width if width is not None else cfg["width"]
    height = height if height is not None else cfg["height"]
    gen = t.Generator(device="cpu")
    gen.manual_seed(seed)
    xy = t.empty(n, 2).uniform_(-1.0, 1.0, generator=gen)
    z = t.empty(n, 1).uniform_(2.0, 6.0, generator=gen)
    mu = t.cat((xy, z), dim=1)
    view = fov_view(width, height, device)
    if cfg.get("clustered"):
        k = int(round(0.8 * n))
        zc = t.empty(k, 1).uniform_(3.0, 3.5, generator=gen)
        half_w = (width / 2.0) / view["fx"]
        half_h = (height / 2.0) / view["fy"]
        xc = t.empty(k, 1).uniform_(-1.0, 1.0, generator=gen) * half_w * zc
        yc = t.empty(k, 1).uniform_(-1.0, 1.0, generator=gen) * half_h * zc
        mu[:k] = t.cat((xc, yc, zc), dim=1)
    if cfg.get("anisotropic"):
        s = t.empty(n, 3).normal_(-5.0, 0.5, generator=gen)
        axis = t.randint(0, 3, (n,), generator=gen)
        big = t.empty(n).normal_(-2.0, 0.5, generator=gen)
        s[t.arange(n), axis] = big
        alpha = t.empty(n, 1).normal_(-1.0, 1.0, generator=gen)
    else:
        s = t.empty(n, 3).normal_(-4.0, 0.5, generator=gen)
        alpha = t.empty(n, 1).normal_(0.0, 1.0, generator=gen)
    q = t.empty(n, 4).normal_(0.0, 1.0, generator=gen)
    q = q / q.norm(dim=1, keepdim=True)
    if cfg["sh"] == "dc":
        rgb = t.empty(n, 3).uniform_(0.0, 1.0, generator=gen)
        A = (rgb - 0.5) / SH_C0
        k_j = t.zeros(n, 15, 3)
    else:
        A = t.empty(n, 3).uniform_(0.0, 1.0, generator=gen)
        k_j = t.empty(n, 15, 3).normal_(0.0, 0.1, generator=gen)
    g = gaussian(n)
    g.mu, g.q, g.s, g.alpha, g.A, g.k_j = mu, q, s, alpha, A, k_j
    return Scene(_finish(g, device, requires_grad), view, f"{name}_{n}_{width}x{height}")


def grad_image(height: int, width: int, device="cpu", seed: int = 1) -> t.Tensor:
    """dL/dimg ~ N(0, 1), seeded on the CPU."""
    gen = t.Generator(device="cpu")
    gen.manual_seed(seed)
    return t.empty(height, width, 3).normal_(0.0, 1.0, generator=gen).to(device)
