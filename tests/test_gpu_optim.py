"""GPU parity of the trainer's optimizer step (the reference's utils/optim.py:12-31
with the clamps of scripts/train.py:171-176 and utils/adc.py:90-93) against
torch.optim.Adam on the device with its default settings (the multi-tensor
path the reference's trainer runs) and against the C++ oracle
(oracle/gs_oracle.cpp, orc_adam_step_f32, its device path).

Bars, per step over 10 steps from the same state: the parameter and both
moments bit for bit equal to torch's on the device, and to the oracle's."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SHAPES = {"mu": (3,), "q": (4,), "Scale": (3,), "Opacity": (1,), "Albedo Coefficient": (3,),
          "Illumination Coefficients": (15, 3)}
LRS = {"mu": 1.6e-4, "q": 1e-3, "Scale": 5e-3, "Opacity": 5e-2, "Albedo Coefficient": 2.5e-3,
       "Illumination Coefficients": 6.25e-4}


def _groups(n, device, seed):
    gen = torch.Generator().manual_seed(seed)
    out = []
    for name, shp in SHAPES.items():
        p = torch.randn((n,) + shp, generator=gen) * (4.0 if name == "Opacity" else 1.0)
        out.append((name, p))
    return out


@pytest.mark.parametrize("n", [100_003, 1, 7, 1001])
def test_fused_adam_matches_torch_adam(device, n):
    from gaussian_splatting.utils.optim import FusedAdam, set_trainer_clamps

    print(f"[gpu] fused Adam, {n} Gaussians", flush=True)
    groups = _groups(n, device, seed=n)
    ours = [torch.nn.Parameter(p.clone().to(device)) for _, p in groups]
    ref = [torch.nn.Parameter(p.clone().to(device)) for _, p in groups]
    opt = FusedAdam([{"params": [p], "lr": LRS[nm], "name": nm}
                     for p, (nm, _) in zip(ours, groups)], lr=0.01, eps=1e-15)
    set_trainer_clamps(opt, scene_extent=0.6)
    topt = torch.optim.Adam([{"params": [p], "lr": LRS[nm], "name": nm}
                             for p, (nm, _) in zip(ref, groups)], lr=0.01, eps=1e-15)
    lo_op, hi_op = math.log(1e-4 / (1 - 1e-4)), math.log(0.99 / 0.01)
    hi_s = math.log(max(0.1 * 0.6, 1e-7))
    gen = torch.Generator().manual_seed(100 + n)
    for step in range(1, 11):
        for po, pr in zip(ours, ref):
            g = torch.randn(pr.shape, generator=gen) * float(10.0 ** (-6 + 7 * torch.rand(1, generator=gen)))
            g[::17] = 0.0
            pr.grad = g.to(device)
            po.grad = g.to(device)
        opt.step()
        topt.step()
        with torch.no_grad():
            ref[3].clamp_(lo_op, hi_op)   # Opacity (train.py:171-176)
            ref[2].clamp_(max=hi_s)       # Scale (adc.py:90-93)
        for i, ((nm, _), po, pr) in enumerate(zip(groups, ours, ref)):
            so, sr = opt.state[po], topt.state[pr]
            assert float(so["step"]) == float(sr["step"]) == step
            for key in ("exp_avg", "exp_avg_sq"):
                a, b = so[key].cpu().numpy(), sr[key].cpu().numpy()
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{nm} {key} step {step}"
            a, b = po.detach().cpu().numpy(), pr.detach().cpu().numpy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{nm} param step {step}"
        # resynchronise to torch's state so every step is compared from the same inputs
        with torch.no_grad():
            for po, pr in zip(ours, ref):
                po.copy_(pr)
                opt.state[po]["exp_avg"].copy_(topt.state[pr]["exp_avg"])
                opt.state[po]["exp_avg_sq"].copy_(topt.state[pr]["exp_avg_sq"])


def test_fused_adam_equals_the_oracle_bitwise(crc, device):
    rng = np.random.default_rng(3)
    n = 250_001
    p = rng.normal(size=n).astype(np.float32)
    m = rng.normal(scale=1e-3, size=n).astype(np.float32)
    v = np.abs(rng.normal(scale=1e-6, size=n)).astype(np.float32)
    g = (rng.normal(size=n) * 10.0 ** rng.uniform(-8, 2, n)).astype(np.float32)
    g[::11] = 0.0
    for step, lr, lo, hi in ((1, 1e-3, -np.inf, np.inf), (7, 5e-2, -0.5, 0.25), (1000, 1.6e-4, -np.inf, 0.1)):
        want = orc.adam_step(p, g, m, v, lr, step, clamp_min=lo, clamp_max=hi)
        t = [torch.from_numpy(x.copy()).to(device) for x in (p, g, m, v)]
        crc.adam_step([t[0]], [t[1]], [t[2]], [t[3]], [lr], [step], [float(lo)], [float(hi)],
                      0.9, 0.999, 1e-15)
        got = [t[0].cpu().numpy(), t[2].cpu().numpy(), t[3].cpu().numpy()]
        for a, b, nm in zip(got, want, ("param", "exp_avg", "exp_avg_sq")):
            same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
            assert same.all(), f"{nm} step {step}: {(~same).sum()} differ"


def test_fused_adam_with_the_reference_scheduler(device):
    """setup_optimizer + get_positional_lr_scheduler as the reference's trainer
    builds them (train.py:106-140): the same groups, names and learning rates
    over steps as torch.optim.Adam with the same scheduler."""
    from gaussian_splatting.scene.gaussian import gaussian
    from gaussian_splatting.utils.optim import (get_mu_lr, get_positional_lr_scheduler,
                                                get_scale_lr, setup_optimizer)

    g = gaussian(1000)
    for k, shp in (("mu", (3,)), ("q", (4,)), ("s", (3,)), ("alpha", (1,)), ("A", (3,)),
                   ("k_j", (15, 3))):
        setattr(g, k, torch.randn((1000,) + shp, device=device))
    lrs = {"mu": 1e-4, "q": 1e-3, "s": 5e-3, "alpha": 5e-2, "A": 2.5e-3, "k_j": 6.25e-4}
    opt = setup_optimizer(g, lrs)
    assert [gr["name"] for gr in opt.param_groups] == list(SHAPES)
    sched = get_positional_lr_scheduler(opt, lr_init=1e-4, lr_final=1e-6, max_steps=50)
    seen = []
    for _ in range(5):
        for p in (g.mu, g.q, g.s, g.alpha, g.A, g.k_j):
            p.grad = torch.ones_like(p)
        opt.step()
        sched.step()
        seen.append((get_mu_lr(opt), get_scale_lr(opt)))
    # the log-linear decay: lr(step) = lr_init (lr_final / lr_init)^(step / max_steps)
    for k, (mu_lr, s_lr) in enumerate(seen, start=1):
        assert mu_lr == pytest.approx(1e-4 * (1e-2) ** (k / 50), rel=1e-12)
        assert s_lr == pytest.approx(5e-3 * (1e-2) ** (k / 50), rel=1e-12)
    assert opt.param_groups[1]["lr"] == 1e-3
