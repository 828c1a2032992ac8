"""Adaptive density control, counterpart of the reference's
gaussian_splatting/utils/adc.py (same functions, arguments, buffers on the
gaussian, optimizer-state handling and returned statistics), on HIP kernels.

- ``accumulate_densification_stats`` / ``update_max_radii2d`` (adc.py:58-87):
  one elementwise kernel (``custom_rasterizer_cuda.adc_stats``);
  ``densification_stats`` does both in one launch.
- ``adaptive_density_control`` (adc.py:316-393): one plan kernel decides every
  Gaussian's fate (clone, split, prune of each copy it would add), one scan
  places the survivors, one gather writes the new cloud and both Adam moments in
  the reference's order; the split copies' N(0, 1) draws come from torch's
  generator exactly as the reference's ``torch.normal`` takes them.  The
  optimizer's groups and state are rebound as the reference's
  ``update_optimizer_state`` (adc.py:122-165) leaves them.  There is no
  fallback path.
"""

from __future__ import annotations

import importlib
import math

import torch as t
from torch.nn import Parameter

from gaussian_splatting.scene.gaussian import gaussian

_glue = importlib.import_module("gaussian_splatting.rasterizer.rasterize")

_GROUP_TO_ATTR = {
    "mu": "mu",
    "q": "q",
    "Scale": "s",
    "Opacity": "alpha",
    "Albedo Coefficient": "A",
    "Illumination Coefficients": "k_j",
}
_ATTRS = ("mu", "q", "s", "alpha", "A", "k_j")


def _crc():
    if _glue.crc is None:
        raise ImportError("custom_rasterizer_cuda is not built. "
                          "Build it with: python custom-3dgs-cuda_amd/build.py")
    return _glue.crc


def scene_extent_from_means(mu: t.Tensor) -> float:
    """Diagonal of the means' bounding box, at least 1e-3 (adc.py:22-26)."""
    extent = float((mu.max(dim=0).values - mu.min(dim=0).values).norm().item())
    return max(extent, 1e-3)


def scene_extent_from_cameras(cameras) -> float:
    """1.1 x the largest camera-centre distance from their mean, at least 1e-3
    (adc.py:29-33)."""
    centers = -t.bmm(cameras.R.transpose(1, 2).contiguous(), cameras.t.unsqueeze(-1)).squeeze(-1)
    extent = float((centers - centers.mean(dim=0)).norm(dim=-1).max().item()) * 1.1
    return max(extent, 1e-3)


def ensure_densification_state(gaussians: gaussian) -> None:
    """Allocate the densification buffers, or resize them to ``mu``'s length
    keeping their prefix (adc.py:36-55)."""
    n = int(gaussians.mu.shape[0])
    like = gaussians.mu

    def fit(buf, rest):
        if buf is None:
            return t.zeros((n, *rest), device=like.device, dtype=like.dtype)
        if buf.shape[0] == n:
            return buf
        out = t.zeros((n, *rest), device=like.device, dtype=like.dtype)
        k = min(int(buf.shape[0]), n)
        if k > 0:
            out[:k] = buf[:k]
        return out

    gaussians.xyz_grad_accum = fit(getattr(gaussians, "xyz_grad_accum", None), (1,))
    gaussians.denom = fit(getattr(gaussians, "denom", None), (1,))
    gaussians.max_radii2D = fit(getattr(gaussians, "max_radii2D", None), ()).view(n)


def densification_stats(gaussians: gaussian, mean2d_grad: t.Tensor | None = None,
                        radii: t.Tensor | None = None, *, width: int | None = None,
                        height: int | None = None) -> None:
    """accumulate_densification_stats and update_max_radii2d in one launch."""
    n = int(gaussians.mu.shape[0])
    if mean2d_grad is not None and mean2d_grad.shape[0] != n:
        mean2d_grad = None
    if radii is not None and radii.shape[0] != n:
        radii = None
    if mean2d_grad is None and radii is None:
        return
    ensure_densification_state(gaussians)
    g = None if mean2d_grad is None else mean2d_grad.detach()[:, :2].float().contiguous()
    r = None if radii is None else radii.detach().float().reshape(n).contiguous()
    w = int(width) if (width is not None and height is not None and width > 0 and height > 0) else 0
    h = int(height) if w else 0
    _crc().adc_stats(g, w, h, r, gaussians.xyz_grad_accum, gaussians.denom,
                     gaussians.max_radii2D)


def accumulate_densification_stats(gaussians: gaussian, mean2d_grad: t.Tensor | None = None, *,
                                   width: int | None = None, height: int | None = None) -> None:
    """adc.py:58-74: the norm of the mean2d gradient, scaled by (W/2, H/2),
    added to xyz_grad_accum and 1 to denom where it is above zero."""
    densification_stats(gaussians, mean2d_grad, None, width=width, height=height)


def update_max_radii2d(gaussians: gaussian, radii: t.Tensor | None) -> None:
    """adc.py:77-81: max_radii2D = max(max_radii2D, radii)."""
    densification_stats(gaussians, None, radii)


def clamp_log_scales(gaussians: gaussian, scene_extent: float) -> None:
    """adc.py:84-86: log-scales at most log(max(0.1 extent, 1e-7))."""
    gaussians.s.data.clamp_(max=math.log(max(0.1 * scene_extent, 1e-7)))


def _rebind(gaussians: gaussian, optimizer: t.optim.Optimizer, cloud: dict,
            moments: dict) -> None:
    """Put the new cloud and its moments in the optimizer's groups and state
    (what the reference's update_optimizer_state leaves there, adc.py:122-165:
    per-element state rewritten, the step count kept) and on the gaussian
    (adc.py:168-171)."""
    for group in optimizer.param_groups:
        attr = _GROUP_TO_ATTR[group["name"]]
        old = group["params"][0]
        stored = optimizer.state.get(old, None)
        param = Parameter(cloud[attr])
        group["params"][0] = param
        if stored is not None:
            state = dict(stored)
            m, v = moments[attr]
            if m is not None:
                state["exp_avg"] = m
            if v is not None:
                state["exp_avg_sq"] = v
            del optimizer.state[old]
            optimizer.state[param] = state
    for group in optimizer.param_groups:
        setattr(gaussians, _GROUP_TO_ATTR[group["name"]], group["params"][0])
    gaussians.N = int(gaussians.mu.shape[0])


def adaptive_density_control(
    gaussians: gaussian,
    optimizer: t.optim.Optimizer,
    *,
    grad_threshold: float = 0.00005,
    percent_dense: float = 0.01,
    min_opacity: float = 0.01,
    max_screen_size: float | None = None,
    scene_extent: float | None = None,
    reset_opacity: bool = False,
    max_gaussians: int = 800_000,
    allow_densify: bool = True,
) -> tuple[gaussian, t.optim.Optimizer, dict[str, int]]:
    """Refined adaptive density control (adc.py:316-393): clone small
    Gaussians with large mean-gradient norms, split large ones into two
    perturbed copies at 1/1.6 the scale, prune faint, huge and (with
    max_screen_size) screen-filling ones, optionally reset opacities; the
    densification buffers start again from zero.  Returns (gaussians,
    optimizer, {"cloned", "split", "pruned"})."""
    ensure_densification_state(gaussians)
    if scene_extent is None:
        raise ValueError("scene_extent must be provided.")
    if not allow_densify:
        # no clone, split, prune or reset (adc.py:351-384): the Parameters and
        # the optimizer state stay as they are; the buffers start again
        n = int(gaussians.mu.shape[0])
        gaussians.xyz_grad_accum = t.zeros(n, 1, device=gaussians.mu.device,
                                           dtype=gaussians.mu.dtype)
        gaussians.denom = t.zeros(n, 1, device=gaussians.mu.device, dtype=gaussians.mu.dtype)
        gaussians.max_radii2D.zero_()
        return gaussians, optimizer, {"cloned": 0, "split": 0, "pruned": 0}
    crc = _crc()
    attrs = {_GROUP_TO_ATTR[g["name"]]: g["params"][0] for g in optimizer.param_groups}
    missing = [a for a in _ATTRS if a not in attrs]
    if missing:
        raise ValueError(f"optimizer has no group for {missing}")
    params = [attrs[a].detach().contiguous() for a in _ATTRS]
    n_before = int(params[0].shape[0])
    densify = bool(allow_densify and n_before < max_gaussians)
    cfg = dict(grad_threshold=float(grad_threshold), percent_dense=float(percent_dense),
               scene_extent=float(scene_extent), min_opacity=float(min_opacity),
               max_screen_size=None if max_screen_size is None else float(max_screen_size))

    moments = []
    for which in ("exp_avg", "exp_avg_sq"):
        for a in _ATTRS:
            st = optimizer.state.get(attrs[a], None)
            moments.append(None if st is None or which not in st else st[which].contiguous())
    noise = None

    def run(prune: bool, reset: bool):
        nonlocal noise
        counts, ws = crc.adc_plan(params, gaussians.xyz_grad_accum.reshape(-1),
                                  gaussians.denom.reshape(-1), gaussians.max_radii2D.reshape(-1),
                                  cfg["grad_threshold"], cfg["percent_dense"],
                                  cfg["scene_extent"], cfg["min_opacity"],
                                  cfg["max_screen_size"], densify, prune, reset)
        if noise is None:
            # the split copies' draws, taken once as the reference's torch.normal
            # takes them (2 n_split rows of 3)
            n_src = counts[3]
            noise = (t.randn(2 * n_src, 3, device=params[0].device, dtype=t.float32) if n_src
                     else params[0].new_zeros(1))
        n_out = counts[0] + counts[1] + 2 * counts[2]
        out, mout = crc.adc_apply(params, moments, noise, ws, n_out, cfg["grad_threshold"],
                                  cfg["percent_dense"], cfg["scene_extent"], cfg["min_opacity"],
                                  cfg["max_screen_size"], densify, prune, reset)
        cloud = dict(zip(_ATTRS, out))
        mom = {a: (mout[i], mout[6 + i]) for i, a in enumerate(_ATTRS)}
        return counts, cloud, mom

    counts, cloud, mom = run(prune=bool(allow_densify), reset=bool(reset_opacity and allow_densify))
    n_clone, n_split = counts[4], counts[3]
    n_post = n_before + n_clone + n_split
    n_out = counts[0] + counts[1] + 2 * counts[2]
    n_pruned = n_post - n_out if allow_densify else 0
    if allow_densify and n_out == 0 and n_post > 0:
        # every Gaussian pruned: keep the most opaque tenth (adc.py:380-386) of
        # the densified cloud (rebuilt unpruned with the same draws)
        counts, cloud, mom = run(prune=False, reset=False)
        opacity = t.sigmoid(cloud["alpha"].squeeze(-1))
        keep_n = max(1, n_post // 10)
        keep = t.zeros(n_post, dtype=t.bool, device=opacity.device)
        keep[t.topk(opacity, k=keep_n).indices] = True
        cloud = {a: v[keep] for a, v in cloud.items()}
        mom = {a: tuple(None if x is None else x[keep] for x in mv) for a, mv in mom.items()}
        n_pruned = n_post - keep_n
        if reset_opacity:
            cloud["alpha"] = t.clamp_max(cloud["alpha"], math.log(0.01 / (1.0 - 0.01)))
            mom["alpha"] = tuple(None if x is None else t.zeros_like(x) for x in mom["alpha"])
    _rebind(gaussians, optimizer, cloud, mom)
    n = int(gaussians.mu.shape[0])
    gaussians.xyz_grad_accum = t.zeros(n, 1, device=gaussians.mu.device, dtype=gaussians.mu.dtype)
    gaussians.denom = t.zeros(n, 1, device=gaussians.mu.device, dtype=gaussians.mu.dtype)
    gaussians.max_radii2D = t.zeros(n, device=gaussians.mu.device, dtype=gaussians.mu.dtype)
    return gaussians, optimizer, {"cloned": int(n_clone), "split": int(n_split),
                                  "pruned": int(n_pruned)}
