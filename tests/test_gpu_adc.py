"""GPU parity of adaptive density control (gaussian_splatting/utils/adc.py of the
reference) against the oracle (oracle/adc_oracle.py, pinned in
test_oracle_adc.py), with the same N(0, 1) draws for the split copies (the
device generator reseeded and drawn again as the pass draws it).

Bars: the statistics bit for bit; the counts equal; every copied value of the
new cloud (all of q, alpha, A, k_j; mu and s of survivors and clones) and both
Adam moments bit for bit, which also pins the reference's order; the split
copies' mu within 2e-6 and s within 4 ulp (exp, log and the rotation product
are the device's, not numpy's)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splatting.scene.gaussian import gaussian
from oracle import adc_oracle as ao
from test_oracle_adc import _cloud

pytestmark = pytest.mark.gpu
NAMES = ao.NAMES


def test_densification_stats_bitwise(device):
    from gaussian_splatting.utils.adc import densification_stats

    rng = np.random.default_rng(0)
    n = 100_003
    g = gaussian(n)
    g.mu = torch.zeros(n, 3, device=device)
    grad = rng.normal(size=(n, 2)).astype(np.float32) * 1e-3
    grad[::7] = 0.0
    grad[3, 1] = np.nan
    radii = np.abs(rng.normal(size=n)).astype(np.float32) * 9
    radii[5] = np.nan
    acc = np.abs(rng.normal(size=n)).astype(np.float32)
    den = rng.integers(0, 5, n).astype(np.float32)
    mr = np.abs(rng.normal(size=n)).astype(np.float32) * 9
    g.xyz_grad_accum = torch.from_numpy(acc.reshape(n, 1)).to(device)
    g.denom = torch.from_numpy(den.reshape(n, 1)).to(device)
    g.max_radii2D = torch.from_numpy(mr).to(device)
    densification_stats(g, torch.from_numpy(grad).to(device), torch.from_numpy(radii).to(device),
                        width=1920, height=1080)
    wa, wd, wr = ao.stats(acc, den, mr, grad, radii, width=1920, height=1080)
    for got, want, nm in ((g.xyz_grad_accum, wa, "accum"), (g.denom, wd, "denom"),
                          (g.max_radii2D, wr, "max_radii2D")):
        a = got.cpu().numpy().reshape(-1)
        same = (a.view(np.uint32) == want.view(np.uint32)) | (np.isnan(a) & np.isnan(want))
        assert same.all(), nm


def _setup(device, n, seed, with_state=True):
    from gaussian_splatting.utils.optim import FusedAdam

    c, m, accum, denom, maxr = _cloud(n, seed)
    g = gaussian(n)
    params = {}
    for k, attr in zip(NAMES, NAMES):
        params[k] = torch.nn.Parameter(torch.from_numpy(c[k]).to(device))
        setattr(g, attr, params[k])
    groups = [{"params": [params[k]], "lr": 1e-3, "name": nm} for k, nm in
              zip(NAMES, ("mu", "q", "Scale", "Opacity", "Albedo Coefficient",
                          "Illumination Coefficients"))]
    opt = FusedAdam(groups, lr=0.01, eps=1e-15)
    if with_state:
        for k in NAMES:
            st = opt.state[params[k]]
            st["step"] = torch.tensor(3.0)
            st["exp_avg"] = torch.from_numpy(m[k][0]).to(device)
            st["exp_avg_sq"] = torch.from_numpy(m[k][1]).to(device)
    g.xyz_grad_accum = torch.from_numpy(accum.reshape(n, 1)).to(device)
    g.denom = torch.from_numpy(denom.reshape(n, 1)).to(device)
    g.max_radii2D = torch.from_numpy(maxr).to(device)
    return g, opt, c, (m if with_state else None), accum, denom, maxr


@pytest.mark.parametrize("n,seed,reset,screen", [(20_000, 1, False, 40.0), (20_000, 2, True, None),
                                                  (4097, 3, False, 40.0), (1, 4, False, None)])
def test_adc_matches_the_oracle(device, n, seed, reset, screen):
    from gaussian_splatting.utils.adc import adaptive_density_control

    g, opt, c, m, accum, denom, maxr = _setup(device, n, seed)
    torch.manual_seed(1234)
    g, opt, st = adaptive_density_control(g, opt, scene_extent=5.0, max_screen_size=screen,
                                          reset_opacity=reset)
    torch.manual_seed(1234)
    ns = st["split"]
    z = torch.randn(2 * ns, 3, device=device).cpu().numpy() if ns else None
    want, wm, wst = ao.adc(c, m, accum, denom, maxr, z, scene_extent=5.0, max_screen_size=screen,
                           reset_opacity=reset)
    assert st == wst
    got = {k: getattr(g, k).detach().cpu().numpy() for k in NAMES}
    n_out = want["mu"].shape[0]
    assert g.N == n_out and g.xyz_grad_accum.shape == (n_out, 1) and g.max_radii2D.shape == (n_out,)
    for k in ("q", "alpha", "A", "k_j"):
        assert np.array_equal(got[k].view(np.uint32), want[k].view(np.uint32)), k
    # mu and s: bit for bit except the split copies (a tail of the cloud)
    eq_mu = np.all(got["mu"] == want["mu"], axis=1)
    eq_s = np.all(got["s"] == want["s"], axis=1)
    first = int(np.argmin(eq_mu & eq_s)) if not (eq_mu & eq_s).all() else n_out
    assert (eq_mu & eq_s)[:first].all()
    assert np.allclose(got["mu"][first:], want["mu"][first:], rtol=2e-6, atol=2e-6)
    ds = np.abs(got["s"][first:].view(np.int32).astype(np.int64) - want["s"][first:].view(np.int32))
    assert ds.size == 0 or ds.max() <= 4
    for i, k in enumerate(NAMES):
        st_ = opt.state[opt.param_groups[i]["params"][0]]
        assert float(st_["step"]) == 3.0
        for j, key in enumerate(("exp_avg", "exp_avg_sq")):
            assert np.array_equal(st_[key].cpu().numpy(), wm[k][j]), (k, key)
    assert opt.param_groups[0]["params"][0] is g.mu


def test_adc_all_pruned_and_no_state(device):
    from gaussian_splatting.utils.adc import adaptive_density_control

    g, opt, c, _, accum, denom, maxr = _setup(device, 500, 7, with_state=False)
    with torch.no_grad():
        g.alpha.copy_(torch.linspace(-9, -6, 500, device=device)[:, None])
    c["alpha"] = g.alpha.detach().cpu().numpy()
    accum[:] = 0.0
    g.xyz_grad_accum.zero_()
    g, opt, st = adaptive_density_control(g, opt, scene_extent=5.0, reset_opacity=True)
    want, _, wst = ao.adc(c, None, accum, denom, maxr, None, scene_extent=5.0, reset_opacity=True)
    assert st == wst == {"cloned": 0, "split": 0, "pruned": 450}
    for k in NAMES:
        assert np.array_equal(getattr(g, k).detach().cpu().numpy(), want[k]), k
    assert len(opt.state) == 0


def test_adc_without_densify_leaves_the_cloud_untouched(device):
    """allow_densify=False (the reference's frozen topology, adc.py:351-384):
    the same Parameter objects and optimizer state, values unchanged, only the
    densification buffers restarted; the oracle agrees."""
    from gaussian_splatting.utils.adc import adaptive_density_control

    g, opt, c, m, accum, denom, maxr = _setup(device, 2000, 5)
    params = {k: getattr(g, k) for k in NAMES}
    before = {k: v.detach().clone() for k, v in params.items()}
    states = {k: dict(opt.state[v]) for k, v in params.items()}
    radii = g.max_radii2D.data_ptr()
    g, opt, st = adaptive_density_control(g, opt, scene_extent=5.0, reset_opacity=True,
                                          allow_densify=False)
    want, _, wst = ao.adc(c, m, accum, denom, maxr, None, scene_extent=5.0, reset_opacity=True,
                          allow_densify=False)
    assert st == wst == {"cloned": 0, "split": 0, "pruned": 0}
    for k in NAMES:
        assert getattr(g, k) is params[k]
        assert torch.equal(getattr(g, k).detach(), before[k])
        assert np.array_equal(getattr(g, k).detach().cpu().numpy(), want[k]), k
        for key in ("exp_avg", "exp_avg_sq"):
            assert opt.state[params[k]][key] is states[k][key]
    # cleared in place, as the reference's max_radii2D.zero_()
    assert g.max_radii2D.data_ptr() == radii and not g.max_radii2D.any()
    assert not g.xyz_grad_accum.any() and not g.denom.any()
