"""Pins of the optimizer-step oracle (oracle/gs_oracle.cpp, orc_adam_step_f32)
against torch.optim.Adam on CPU (the single-tensor path, the arithmetic torch
documents in torch/optim/adam.py): over 10 steps from the same state, the
moments bit for bit; the parameter within 4 ulps of max(|p|, |update|) (torch's
CPU addcdiv kernel rounds ~0.1% of elements differently from the formula it
documents, by up to ~3 such ulps); and the clamps as torch's clamp_.  The
oracle's device path (torch's multi-tensor path on the GPU, which the trainer
runs and the kernel follows; pinned bit for bit against torch on the GPU in
tests/test_gpu_optim.py) differs from the CPU path only in rounding: the first
moment bit for bit, the second within 2 ulps (the two roundings of
(1 - b2) g g), the parameter within the same 4 ulps."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_adam_oracle_matches_torch(seed):
    rng = np.random.default_rng(seed)
    torch.manual_seed(seed)
    n = 50_003
    p0 = torch.randn(n) * float(10 ** rng.uniform(-3, 0))
    lr = float(10 ** rng.uniform(-5, -1))
    par = torch.nn.Parameter(p0.clone())
    opt = torch.optim.Adam([par], lr=lr, eps=1e-15, foreach=False)
    p, m, v = p0.numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    differ = 0
    for step in range(1, 11):
        g = (torch.randn(n) * float(10 ** rng.uniform(-8, 2))).float()
        g[::13] = 0.0
        par.grad = g.clone()
        opt.step()
        st = opt.state[par]
        tp, tm, tv = par.detach().numpy(), st["exp_avg"].numpy(), st["exp_avg_sq"].numpy()
        op, om, ov = orc.adam_step(p, g.numpy(), m, v, lr, step, path="cpu")
        dp, dm, dv = orc.adam_step(p, g.numpy(), m, v, lr, step, path="device")
        assert np.array_equal(dm.view(np.uint32), om.view(np.uint32))
        assert np.all(np.abs(dv.view(np.int32).astype(np.int64) - ov.view(np.int32)) <= 2)
        derr = np.abs(dp.astype(np.float64) - op)
        assert np.array_equal(om.view(np.uint32), tm.view(np.uint32)), f"exp_avg step {step}"
        assert np.array_equal(ov.view(np.uint32), tv.view(np.uint32)), f"exp_avg_sq step {step}"
        scale = np.maximum(np.abs(p.astype(np.float64)), np.abs(tp.astype(np.float64) - p))
        err = np.abs(op.astype(np.float64) - tp)
        assert np.all(err <= 4 * 2.0 ** -23 * np.maximum(scale, 1e-38)), f"param step {step}"
        assert np.all(derr <= 4 * 2.0 ** -23 * np.maximum(scale, 1e-38)), f"device param step {step}"
        differ += int((op != tp).sum())
        p, m, v = tp.copy(), tm.copy(), tv.copy()
    assert differ <= 0.005 * 10 * n  # a fraction of a percent of the elements


def test_adam_oracle_clamps_like_torch():
    p = np.array([-3.0, 0.5, 2.0, np.nan, 10.0], np.float32)
    g = np.array([1.0, -1.0, 0.5, 0.1, -2.0], np.float32)
    z = np.zeros(5, np.float32)
    op, _, _ = orc.adam_step(p, g, z, z, 0.5, 1, clamp_min=-1.0, clamp_max=1.5, path="cpu")
    par = torch.nn.Parameter(torch.from_numpy(p.copy()))
    par.grad = torch.from_numpy(g.copy())
    opt = torch.optim.Adam([par], lr=0.5, eps=1e-15, foreach=False)
    opt.step()
    want = par.detach().clamp_(-1.0, 1.5).numpy()
    assert np.array_equal(np.isnan(op), np.isnan(want))
    assert np.array_equal(op[~np.isnan(op)], want[~np.isnan(want)])
