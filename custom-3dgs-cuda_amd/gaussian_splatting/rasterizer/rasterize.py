"""Autograd glue over ``custom_rasterizer_cuda`` — the counterpart of the reference's
gaussian_splatting/rasterizer/rasterize.py:10-160, same call order and semantics:

forward:  cam_position = -R^T t; project -> (mean2d, cov2d, depth); approximate screen
          radii for densification; SH colours (these four in one kernel,
          ``project_sh``, bit for bit the separate ops); rasterize -> image.
backward: backwards_rasterization -> (d mean2d, d cov2d, d colours, d alpha);
          backwards_SH -> (d albedo, d k_j, d mu via view direction);
          backwards_projection -> (d mu, d q, d log-scale); d mu = sum of both paths
          (these three in one kernel, ``backwards_project_sh``, bit for bit the
          separate ops and the sum).

The extension is the MI355X HIP build (libgsraster.so); there is no fallback path.
"""

from __future__ import annotations

import sys
from pathlib import Path

import torch as t

from gaussian_splatting.scene.gaussian import gaussian

try:
    import custom_rasterizer_cuda as crc
except ImportError:  # the built module sits beside this package
    _root = str(Path(__file__).resolve().parents[2])
    if _root not in sys.path:
        sys.path.insert(0, _root)
    try:
        import custom_rasterizer_cuda as crc
    except ImportError:
        crc = None


def _forward(ctx, logits, mu, q, s, alpha_in, albedo, k_j, cam_rotation, cam_translation, fx,
             fy, cx, cy, height, width):
    """The forward of both Functions below; alpha_in is the opacity, or its
    logits when ``logits`` (the sigmoid then runs in the fused head kernel)."""
    if crc is None:
        raise ImportError(
            "custom_rasterizer_cuda is not built. "
            "Build it with: python custom-3dgs-cuda_amd/build.py"
        )

    num_gaussians = mu.shape[0]
    mu = mu.contiguous()
    q = q.contiguous()
    s = s.contiguous()
    alpha_in = alpha_in.contiguous()
    albedo = albedo.contiguous()
    k_j = k_j.contiguous()
    cam_rotation = cam_rotation.contiguous()
    cam_translation = cam_translation.contiguous()

    fx_f, fy_f = float(fx), float(fy)
    cx_f, cy_f = float(cx), float(cy)
    img_h, img_w = int(height), int(width)

    # -R^T t, project, the screen radius ~ 3 * sqrt(max eigenvalue of
    # [[a, b], [b, c]]) and SH (rasterize.py:42-54), the same fp32 operations
    # in one kernel; with logits also t.sigmoid (rasterize.py:149)
    mean_2d, cov_2d, depths, radii, colors, cam_position, opacity = crc.project_sh(
        num_gaussians, mu, q, s, cam_rotation, cam_translation, fx_f, fy_f, cx_f, cy_f,
        albedo, k_j, alpha_in if logits else None
    )
    alpha = opacity if logits else alpha_in
    RasterizeFunction.last_radii2d = radii

    rendered_img, sorted_ids, tile_ranges, final_T, n_contrib = crc.rasterize(
        num_gaussians, depths, mean_2d, cov_2d, colors, alpha, img_h, img_w
    )

    ctx.save_for_backward(
        mean_2d, cov_2d, colors, alpha,
        sorted_ids, tile_ranges, final_T, n_contrib,
        mu, q, s, albedo, k_j,
        cam_rotation, cam_translation, cam_position,
    )
    ctx.logits = logits
    ctx.num_gaussians = num_gaussians
    ctx.height = img_h
    ctx.width = img_w
    ctx.fx = fx_f
    ctx.fy = fy_f
    ctx.cx = cx_f
    ctx.cy = cy_f
    return rendered_img


def _backward(ctx, grad_output):
    (
        mean_2d, cov_2d, colors, alpha,
        sorted_ids, tile_ranges, final_T, n_contrib,
        mu, q, s, albedo, k_j,
        cam_rotation, cam_translation, cam_position,
    ) = ctx.saved_tensors

    # the reference copies grad_output with .contiguous() (rasterize.py:85-86);
    # the strided op reads any [H, W, 3] view in place (image.sum() hands
    # in a broadcast one)
    mean_2d_grad, cov_2d_grad, colors_grad, alpha_grad = crc.backwards_rasterization_strided(
        grad_output, mean_2d, cov_2d, colors, alpha,
        sorted_ids, tile_ranges, final_T, n_contrib,
        ctx.num_gaussians, ctx.height, ctx.width,
    )
    RasterizeFunction.last_mean2d_grad = mean_2d_grad.detach()

    # backwards_SH, backwards_projection and mu_grad + mu_sh_grad
    # (rasterize.py:100-117) in one kernel; with logits also the sigmoid's
    # backward
    mu_grad, q_grad, s_grad, albedo_grad, k_j_grad, logit_grad = crc.backwards_project_sh(
        mean_2d_grad, cov_2d_grad, colors_grad, mu, q, s, cam_rotation, cam_translation,
        ctx.fx, ctx.fy, albedo, k_j, cam_position,
        alpha_grad if ctx.logits else None, alpha if ctx.logits else None,
    )
    # alpha arrives as [N] or [N, 1]; hand back a gradient of the same shape
    alpha_in_grad = logit_grad if ctx.logits else alpha_grad.reshape(alpha.shape)

    return (mu_grad, q_grad, s_grad, alpha_in_grad, albedo_grad, k_j_grad,
            None, None, None, None, None, None, None, None)


class RasterizeFunction(t.autograd.Function):
    """Full rasterization pipeline. Returns the rendered image [H, W, 3].

    After forward, ``last_radii2d`` holds approximate screen radii (N,).
    After backward, ``last_mean2d_grad`` holds dL/d mean2d (N, 2) for densification.
    """

    last_mean2d_grad: t.Tensor | None = None
    last_radii2d: t.Tensor | None = None

    @staticmethod
    def forward(ctx, mu, q, s, alpha, albedo, k_j, cam_rotation, cam_translation, fx, fy, cx, cy,
                height, width):
        return _forward(ctx, False, mu, q, s, alpha, albedo, k_j, cam_rotation, cam_translation,
                        fx, fy, cx, cy, height, width)

    @staticmethod
    def backward(ctx, grad_output):
        return _backward(ctx, grad_output)


class _RasterizeLogitsFunction(t.autograd.Function):
    """RasterizeFunction taking opacity logits: t.sigmoid(alpha) and its
    backward run inside the fused head and tail kernels, bit for bit torch's."""

    @staticmethod
    def forward(ctx, mu, q, s, alpha_logits, albedo, k_j, cam_rotation, cam_translation, fx, fy,
                cx, cy, height, width):
        return _forward(ctx, True, mu, q, s, alpha_logits, albedo, k_j, cam_rotation,
                        cam_translation, fx, fy, cx, cy, height, width)

    @staticmethod
    def backward(ctx, grad_output):
        return _backward(ctx, grad_output)


def rasterize(gaussians: gaussian, image: dict) -> t.Tensor:
    """Training-loop entry point (rasterize.py:137-160).

    Opacity is stored as logits; the sigmoid is applied (in the fused head kernel,
    bit for bit t.sigmoid) so the rasterizer receives opacity in (0, 1) while
    gradients still flow to ``gaussians.alpha``.
    """
    RasterizeFunction.last_mean2d_grad = None
    RasterizeFunction.last_radii2d = None
    return _RasterizeLogitsFunction.apply(
        gaussians.mu,
        gaussians.q,
        gaussians.s,
        gaussians.alpha,
        gaussians.A,
        gaussians.k_j,
        image["R"],
        image["T"],
        image["fx"],
        image["fy"],
        image["cx"],
        image["cy"],
        image["height"],
        image["width"],
    )
