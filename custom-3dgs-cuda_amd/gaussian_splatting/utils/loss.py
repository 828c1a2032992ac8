"""The trainer's reconstruction loss, counterpart of the reference's
gaussian_splatting/utils/loss.py:12-33 (same names, arguments, shape check and
value): (1 - lambda) * mean|gt - rendered| + lambda * (1 - SSIM), the SSIM on
both images clamped to [0, 1] with torchmetrics' defaults (11 x 11 Gaussian
window, sigma 1.5, data range 1).

Both passes are HIP kernels of libgsraster.so (``custom_rasterizer_cuda.l1_dssim``
and ``l1_dssim_backward``): the forward returns the loss on the device and
keeps the SSIM index's derivative maps for the backward, which forms
dL/drendered in one more pass.  No gradient is formed for ``gt_img`` (the
reference's trainer loads it from disk).  There is no fallback path.
"""

from __future__ import annotations

import importlib

import torch as t

# the glue module (the package re-exports its function `rasterize` under the
# same name, so it is looked up by its module name)
_glue = importlib.import_module("gaussian_splatting.rasterizer.rasterize")

LAMBDA_DSSIM = 0.2


def _crc():
    if _glue.crc is None:
        raise ImportError("custom_rasterizer_cuda is not built. "
                          "Build it with: python custom-3dgs-cuda_amd/build.py")
    return _glue.crc


class _L1DSSIM(t.autograd.Function):
    @staticmethod
    def forward(ctx, rendered, gt, lambda_dssim):
        crc = _crc()
        rendered, gt = rendered.contiguous(), gt.contiguous()
        out, ws = crc.l1_dssim(rendered, gt, float(lambda_dssim))
        ctx.save_for_backward(rendered, gt, ws)
        ctx.lambda_dssim = float(lambda_dssim)
        return out[0]

    @staticmethod
    def backward(ctx, grad_loss):
        rendered, gt, ws = ctx.saved_tensors
        g = grad_loss.reshape(1).to(t.float32).contiguous()
        d = _crc().l1_dssim_backward(rendered, gt, ctx.lambda_dssim, ws, g)
        return d, None, None


def calculate_loss(gt_img: t.Tensor, rendered_img: t.Tensor,
                   lambda_dssim: float = LAMBDA_DSSIM) -> t.Tensor:
    """Classic 3DGS reconstruction loss: (1-λ) L1 + λ (1-SSIM) (loss.py:12-33).

    Args:
        gt_img: ground truth (H, W, 3) in [0, 1]
        rendered_img: rendered RGB (H, W, 3)
        lambda_dssim: weight on the D-SSIM term (default 0.2)

    Returns:
        scalar loss (fp32, on the images' device)
    """
    if rendered_img.shape != gt_img.shape:
        raise ValueError(
            f"Shape mismatch: gt {tuple(gt_img.shape)} vs rendered {tuple(rendered_img.shape)}"
        )
    return _L1DSSIM.apply(rendered_img, gt_img.detach(), lambda_dssim)


def ssim(rendered_img: t.Tensor, gt_img: t.Tensor) -> t.Tensor:
    """SSIM of two (H, W, 3) images clamped to [0, 1], as the reference's
    scripts/eval.py:60 scores a view (a 0-d tensor on the device)."""
    if rendered_img.shape != gt_img.shape:
        raise ValueError(
            f"Shape mismatch: gt {tuple(gt_img.shape)} vs rendered {tuple(rendered_img.shape)}"
        )
    # the kernel clamps both images to [0, 1] as it loads them
    return _crc().ssim(rendered_img.detach().contiguous(), gt_img.detach().contiguous())[1]
