"""The trainer's optimizer, counterpart of the reference's
gaussian_splatting/utils/optim.py (same functions, arguments and parameter-group
names), on one HIP kernel per step.

``FusedAdam`` is a ``torch.optim.Optimizer`` with torch.optim.Adam's constructor
arguments, parameter groups and per-parameter state (``step``, ``exp_avg``,
``exp_avg_sq``; the densification code of the reference rewrites that state when
it prunes or grows the parameters, utils/adc.py:122-165), whose ``step()`` runs
the whole update of every group in one launch (libgsraster ``gsr_adam_step``).
Its arithmetic is torch.optim.Adam's default (multi-tensor) path on the
device for fp32 tensors, bit for bit.  A group may
also carry ``clamp_min`` / ``clamp_max``: the updated parameter is clamped in the
same pass, which is how the trainer's clamps after each step
(scripts/train.py:171-176: opacity logits to [logit(1e-4), logit(0.99)];
utils/adc.py:90-93: log-scales to at most log(0.1 extent)) run without a pass
of their own (``set_trainer_clamps``).  There is no fallback path.
"""

from __future__ import annotations

import importlib
import math

import torch as t
from torch.nn import Parameter
from torch.optim.lr_scheduler import LambdaLR

from gaussian_splatting.scene.gaussian import gaussian

_glue = importlib.import_module("gaussian_splatting.rasterizer.rasterize")


def _crc():
    if _glue.crc is None:
        raise ImportError("custom_rasterizer_cuda is not built. "
                          "Build it with: python custom-3dgs-cuda_amd/build.py")
    return _glue.crc


class FusedAdam(t.optim.Optimizer):
    """Adam (no weight decay, no AMSGrad) whose step is one fused HIP kernel
    over every group, with optional per-group clamps of the updated
    parameters (``clamp_min`` / ``clamp_max``, None for none)."""

    def __init__(self, params, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0, clamp_min=None, clamp_max=None):
        if lr < 0.0:
            raise ValueError(f"Invalid learning rate: {lr}")
        if eps < 0.0:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"Invalid beta parameters: {betas}")
        if weight_decay != 0.0:
            raise ValueError("FusedAdam has no weight decay (the trainer uses none)")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=0.0,
                                      clamp_min=clamp_min, clamp_max=clamp_max))

    @t.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with t.enable_grad():
                loss = closure()
        # one launch per (betas, eps) setting; the trainer has one
        batches: dict[tuple, list] = {}
        for group in self.param_groups:
            lo = -math.inf if group.get("clamp_min") is None else float(group["clamp_min"])
            hi = math.inf if group.get("clamp_max") is None else float(group["clamp_max"])
            b1, b2 = group["betas"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("FusedAdam does not support sparse gradients")
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = t.tensor(0.0, dtype=t.float32)
                    state["exp_avg"] = t.zeros_like(p, memory_format=t.preserve_format)
                    state["exp_avg_sq"] = t.zeros_like(p, memory_format=t.preserve_format)
                state["step"] += 1
                batch = batches.setdefault((float(b1), float(b2), float(group["eps"])),
                                           [[] for _ in range(8)])
                for lst, val in zip(batch, (p, p.grad, state["exp_avg"], state["exp_avg_sq"],
                                            float(group["lr"]), int(state["step"].item()), lo,
                                            hi)):
                    lst.append(val)
        for (b1, b2, eps), (ps, gs, ms, vs, lrs, steps, los, his) in batches.items():
            ps_c = [p if p.is_contiguous() else p.contiguous() for p in ps]
            gs = [g.contiguous() for g in gs]
            _crc().adam_step(ps_c, gs, ms, vs, lrs, steps, los, his, b1, b2, eps)
            for p, pc in zip(ps, ps_c):
                if pc is not p:
                    p.copy_(pc)
        return loss


def setup_optimizer(gaussians: gaussian, lrs: dict, lr: float = 0.01) -> FusedAdam:
    """Wrap trainable Gaussian tensors as Parameters and return the fused Adam
    optimizer (utils/optim.py:12-31: same group names, learning rates, eps)."""
    gaussians.mu = Parameter(gaussians.mu.detach())
    gaussians.q = Parameter(gaussians.q.detach())
    gaussians.s = Parameter(gaussians.s.detach())
    gaussians.alpha = Parameter(gaussians.alpha.detach())
    gaussians.A = Parameter(gaussians.A.detach())
    gaussians.k_j = Parameter(gaussians.k_j.detach())
    groups = [
        {"params": [gaussians.mu], "lr": lrs["mu"], "name": "mu"},
        {"params": [gaussians.q], "lr": lrs["q"], "name": "q"},
        {"params": [gaussians.s], "lr": lrs["s"], "name": "Scale"},
        {"params": [gaussians.alpha], "lr": lrs["alpha"], "name": "Opacity"},
        {"params": [gaussians.A], "lr": lrs["A"], "name": "Albedo Coefficient"},
        {"params": [gaussians.k_j], "lr": lrs["k_j"], "name": "Illumination Coefficients"},
    ]
    return FusedAdam(groups, lr=lr, eps=1e-15)


# the trainer's clamps (scripts/train.py:171-176, utils/adc.py:90-93)
OPACITY_LOGIT_MIN = math.log(1e-4 / (1.0 - 1e-4))
OPACITY_LOGIT_MAX = math.log(0.99 / (1.0 - 0.99))


def max_log_scale(scene_extent: float) -> float:
    """utils/adc.py:91: the largest log-scale kept."""
    return math.log(max(0.1 * scene_extent, 1e-7))


def set_trainer_clamps(optimizer: t.optim.Optimizer, scene_extent: float) -> None:
    """Have every step clamp the opacity logits and the log-scales as the
    reference's trainer does after optimizer.step() (train.py:171-176)."""
    for group in optimizer.param_groups:
        if group.get("name") == "Opacity":
            group["clamp_min"], group["clamp_max"] = OPACITY_LOGIT_MIN, OPACITY_LOGIT_MAX
        elif group.get("name") == "Scale":
            group["clamp_min"], group["clamp_max"] = None, max_log_scale(scene_extent)


def clamp_log_scales(gaussians: gaussian, scene_extent: float) -> None:
    """utils/adc.py:90-93 as a separate op (for callers outside the fused step)."""
    gaussians.s.data.clamp_(max=max_log_scale(scene_extent))


def _expon_lr(lr_init: float, lr_final: float, delay_steps: int, delay_mult: float,
              max_steps: int):
    """The multiplier (relative to lr_init) of Inria's get_expon_lr_func:
    log-linear from lr_init to lr_final over max_steps, with an optional
    half-sine warm-up from delay_mult over delay_steps (utils/optim.py:34-60)."""

    def mult(step: int) -> float:
        if lr_init <= 0.0:
            return 0.0
        frac = min(max(step / float(max_steps), 0.0), 1.0)
        lr = math.exp((1.0 - frac) * math.log(lr_init) + frac * math.log(lr_final))
        warm = 1.0
        if delay_steps > 0:
            ramp = min(max(step / float(delay_steps), 0.0), 1.0)
            warm = delay_mult + (1.0 - delay_mult) * math.sin(0.5 * math.pi * ramp)
        return warm * lr / lr_init

    return mult


def get_positional_lr_scheduler(optimizer: t.optim.Optimizer, *, lr_init: float = 1.6e-4,
                                lr_final: float = 1.6e-6, scale_lr_init: float = 5e-3,
                                scale_lr_final: float = 5e-5, lr_delay_steps: int = 0,
                                lr_delay_mult: float = 0.01, max_steps: int = 30_000) -> LambdaLR:
    """Exponential decay of the ``mu`` and ``Scale`` groups' learning rates; the
    other groups keep theirs (utils/optim.py:63-133, same arguments and errors)."""
    if lr_init <= 0.0 or lr_final <= 0.0:
        raise ValueError("lr_init and lr_final must be positive")
    if scale_lr_init <= 0.0 or scale_lr_final <= 0.0:
        raise ValueError("scale_lr_init and scale_lr_final must be positive")
    if max_steps < 1:
        raise ValueError("max_steps must be >= 1")
    index = {g.get("name"): i for i, g in enumerate(optimizer.param_groups)}
    if "mu" not in index:
        raise ValueError("optimizer has no param group named 'mu'")
    if "Scale" not in index:
        raise ValueError("optimizer has no param group named 'Scale'")
    decayed = {index["mu"]: (lr_init, lr_final), index["Scale"]: (scale_lr_init, scale_lr_final)}
    lambdas = []
    for i, group in enumerate(optimizer.param_groups):
        if i in decayed:
            start, end = decayed[i]
            group["lr"] = start
            group["initial_lr"] = start
            lambdas.append(_expon_lr(start, end, lr_delay_steps, lr_delay_mult, max_steps))
        else:
            group.setdefault("initial_lr", group["lr"])
            lambdas.append(lambda _step: 1.0)
    return LambdaLR(optimizer, lr_lambda=lambdas)


def _group_lr(optimizer: t.optim.Optimizer, name: str) -> float:
    for group in optimizer.param_groups:
        if group.get("name") == name:
            return float(group["lr"])
    return float("nan")


def get_mu_lr(optimizer: t.optim.Optimizer) -> float:
    """Current learning rate of the positional (mu) group."""
    return _group_lr(optimizer, "mu")


def get_scale_lr(optimizer: t.optim.Optimizer) -> float:
    """Current learning rate of the Scale group."""
    return _group_lr(optimizer, "Scale")
