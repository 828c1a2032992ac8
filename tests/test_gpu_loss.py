"""GPU parity of the trainer's loss (gaussian_splatting/utils/loss.py:12-33 of the
reference) against the float64 oracle (oracle/loss_oracle.py).

Bars: the loss, SSIM and L1 values within 1e-5 absolute (the fp32 image bar);
dL/drendered within 1e-4 relative (helpers.assert_grad_close: 1e-4 of the
oracle's |value|, floored at 5e-6 of the element's sum of |terms|), with the
tensor's relative error within 1e-4.  Images: rendered ~ N(0.5, 0.35) (some
values outside [0, 1], so the clamp's mask is exercised), gt ~ U[0, 1] plus
exact ties with rendered (the L1 term's zero subgradient)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_grad_close
from oracle import loss_oracle as lo

pytestmark = pytest.mark.gpu


def _pair(H, W, seed):
    rng = np.random.default_rng(seed)
    r = rng.normal(0.5, 0.35, (H, W, 3)).astype(np.float32)
    g = rng.uniform(0.0, 1.0, (H, W, 3)).astype(np.float32)
    tie = rng.random((H, W, 3)) < 0.01
    g[tie] = np.clip(r[tie], 0, 1)
    r[tie] = g[tie]
    return r, g


SIZES = [(11, 11), (37, 53), (256, 256), (270, 480), (1080, 1920)]


@pytest.mark.parametrize("H,W", SIZES, ids=[f"{h}x{w}" for h, w in SIZES])
def test_loss_forward_and_backward(crc, device, H, W):
    print(f"[gpu] loss parity {H}x{W}", flush=True)
    r, g = _pair(H, W, seed=H * 7 + W)
    rt, gt = torch.from_numpy(r).to(device), torch.from_numpy(g).to(device)
    out, ws = crc.l1_dssim(rt, gt, 0.2)
    grad_loss = torch.tensor([1.5], device=device)
    d = crc.l1_dssim_backward(rt, gt, 0.2, ws, grad_loss)
    torch.cuda.synchronize()
    loss, s, l1 = (float(v) for v in out.cpu())
    want = lo.l1_dssim(r, g, 0.2)
    assert abs(loss - want[0]) <= 1e-5 and abs(s - want[1]) <= 1e-5 and abs(l1 - want[2]) <= 1e-5
    wg, ab = lo.l1_dssim_grad(r, g, 0.2, grad_loss=1.5, with_abs=True)
    assert_grad_close(d.cpu().numpy(), wg, ab, f"dL/drendered {H}x{W}")


def test_loss_autograd_function(crc, device):
    """calculate_loss through autograd: loss.backward() gives the kernel's
    gradient, scaled by the upstream gradient; the shape check raises
    ValueError as the reference does."""
    from gaussian_splatting.utils.loss import calculate_loss, ssim

    r, g = _pair(64, 96, seed=3)
    rt = torch.from_numpy(r).to(device).requires_grad_(True)
    gt = torch.from_numpy(g).to(device)
    loss = calculate_loss(gt, rt)
    (3.0 * loss).backward()
    out, ws = crc.l1_dssim(rt.detach(), gt, 0.2)
    d = crc.l1_dssim_backward(rt.detach(), gt, 0.2, ws, torch.tensor([3.0], device=device))
    assert torch.equal(loss.detach(), out[0])
    assert torch.equal(rt.grad, d)
    assert abs(float(ssim(rt, gt)) - lo.ssim(np.clip(r, 0, 1), np.clip(g, 0, 1))) <= 1e-5
    with pytest.raises(ValueError, match="Shape mismatch"):
        calculate_loss(gt[:, :-1], rt)
    with pytest.raises(RuntimeError, match="at least 11 x 11"):
        crc.l1_dssim(rt[:10].contiguous(), gt[:10].contiguous(), 0.2)


def test_loss_is_deterministic(crc, device):
    r, g = _pair(540, 960, seed=9)
    rt, gt = torch.from_numpy(r).to(device), torch.from_numpy(g).to(device)
    o1, w1 = crc.l1_dssim(rt, gt, 0.2)
    d1 = crc.l1_dssim_backward(rt, gt, 0.2, w1)
    o2, w2 = crc.l1_dssim(rt, gt, 0.2)
    d2 = crc.l1_dssim_backward(rt, gt, 0.2, w2)
    assert torch.equal(o1, o2) and torch.equal(d1, d2)
