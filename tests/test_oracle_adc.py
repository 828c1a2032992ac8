"""Pins of the densification oracle (oracle/adc_oracle.py), CPU only, by the
invariants the reference's algorithm (gaussian_splatting/utils/adc.py) fixes:
the statistics' closed form; the count bookkeeping (n + clones + splits - pruned);
the reference's order of the new cloud (survivors, clones, first split copies,
second split copies); clones are exact copies with zero moments; split copies
sit at mu + R(q) (z * exp(s)) with R built independently (scipy's rotation from
the normalized quaternion) and log-scale s - log(1.6); every pruned Gaussian
meets a prune predicate and no survivor does; the all-pruned case keeps the most
opaque tenth; the opacity reset."""

from __future__ import annotations

import math

import numpy as np
import pytest
from scipy.spatial.transform import Rotation

from oracle import adc_oracle as ao

NAMES = ao.NAMES


def _cloud(n, seed):
    rng = np.random.default_rng(seed)
    c = {"mu": rng.normal(size=(n, 3)), "q": rng.normal(size=(n, 4)),
         "s": rng.normal(-4.5, 1.0, (n, 3)), "alpha": rng.normal(0.0, 3.0, (n, 1)),
         "A": rng.uniform(size=(n, 3)), "k_j": rng.normal(0, 0.1, (n, 15, 3))}
    c = {k: v.astype(np.float32) for k, v in c.items()}
    m = {k: (rng.normal(size=c[k].shape).astype(np.float32),
             np.abs(rng.normal(size=c[k].shape)).astype(np.float32)) for k in NAMES}
    accum = np.abs(rng.normal(0, 2e-4, n)).astype(np.float32)
    denom = rng.integers(0, 4, n).astype(np.float32)
    maxr = np.abs(rng.normal(0, 20, n)).astype(np.float32)
    return c, m, accum, denom, maxr


def test_stats_closed_form():
    rng = np.random.default_rng(0)
    n = 1000
    g = rng.normal(size=(n, 2)).astype(np.float32)
    g[::5] = 0.0
    acc0, den0, r0 = (np.zeros(n, np.float32) + 1.0 for _ in range(3))
    radii = np.abs(rng.normal(size=n)).astype(np.float32) * 3
    acc, den, maxr = ao.stats(acc0, den0, r0, g, radii, width=640, height=480)
    nrm = np.hypot(g[:, 0] * 320.0, g[:, 1] * 240.0)
    vis = nrm > 0
    assert np.allclose(acc[vis], 1.0 + nrm[vis], rtol=1e-6) and np.all(acc[~vis] == 1.0)
    assert np.all(den == np.where(vis, 2.0, 1.0))
    assert np.array_equal(maxr, np.maximum(1.0, radii))


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_adc_invariants(seed):
    n, E = 4000, 5.0
    c, m, accum, denom, maxr = _cloud(n, seed)
    den = np.maximum(denom, 1)
    grads = accum / den
    smax = np.exp(c["s"]).max(1)
    clone = (grads >= np.float32(5e-5)) & (smax <= np.float32(0.01 * E))
    split = (grads >= np.float32(5e-5)) & (smax > np.float32(0.01 * E))
    ns = int(split.sum())
    z = np.random.default_rng(seed + 10).normal(size=(2 * ns, 3)).astype(np.float32)
    out, mo, st = ao.adc(c, m, accum, denom, maxr, z, scene_extent=E, max_screen_size=40.0)
    assert st["cloned"] == int(clone.sum()) > 0 and st["split"] == ns > 0
    n_post = n + st["cloned"] + st["split"]
    assert out["mu"].shape[0] == n_post - st["pruned"]
    # the densified cloud before pruning, built from the definitions
    keep_o = ~split
    post = {k: np.concatenate([c[k][keep_o], c[k][clone], c[k][split], c[k][split]])
            for k in NAMES}
    rot = Rotation.from_quat(np.roll(c["q"][split].astype(np.float64), -1, axis=1))
    R = rot.as_matrix()
    sc = np.exp(c["s"][split].astype(np.float64))
    for k in range(2):
        lo = int(keep_o.sum()) + st["cloned"] + k * ns
        zz = z[k * ns:(k + 1) * ns].astype(np.float64)
        post["mu"][lo:lo + ns] = np.einsum("nij,nj->ni", R, zz * sc) + c["mu"][split]
        post["s"][lo:lo + ns] = c["s"][split] - np.log(1.6)
    radii = np.concatenate([maxr[keep_o], np.zeros(st["cloned"] + 2 * ns)])
    op = 1 / (1 + np.exp(-post["alpha"][:, 0].astype(np.float64)))
    prune = (op < 0.01) | (np.exp(post["s"].astype(np.float64)).max(1) > 0.1 * E) | (radii > 40.0)
    assert int(prune.sum()) == st["pruned"]
    for k in NAMES:
        want = post[k][~prune]
        tol = 2e-5 if k in ("mu", "s") else 0.0
        assert np.allclose(out[k], want, rtol=tol, atol=tol), k
    # moments: survivors carry theirs, new Gaussians start at zero
    for k in NAMES:
        for j in range(2):
            full = np.concatenate([m[k][j][keep_o], np.zeros_like(c[k][clone]),
                                   np.zeros_like(c[k][split]), np.zeros_like(c[k][split])])
            assert np.array_equal(mo[k][j], full[~prune]), (k, j)


def test_all_pruned_keeps_the_most_opaque_tenth_and_resets():
    c, m, accum, denom, maxr = _cloud(500, 7)
    c["alpha"][:] = np.linspace(-9, -6, 500, dtype=np.float32)[:, None]  # all below 1% opacity
    accum[:] = 0.0
    out, mo, st = ao.adc(c, m, accum, denom, maxr, np.zeros((0, 3), np.float32), scene_extent=5.0,
                         reset_opacity=True)
    assert st == {"cloned": 0, "split": 0, "pruned": 450}
    assert out["mu"].shape[0] == 50
    assert np.array_equal(out["mu"], c["mu"][450:])  # the largest logits, in index order
    lv = np.float32(math.log(0.01 / 0.99))
    assert np.array_equal(out["alpha"], np.minimum(c["alpha"][450:], lv))
    assert not np.any(mo["alpha"][0]) and not np.any(mo["alpha"][1])


def test_no_densify_past_the_cap_and_window():
    c, m, accum, denom, maxr = _cloud(300, 8)
    out, _, st = ao.adc(c, m, accum, denom, maxr, None, scene_extent=5.0, max_gaussians=300)
    assert st["cloned"] == 0 and st["split"] == 0
    out2, _, st2 = ao.adc(c, m, accum, denom, maxr, None, scene_extent=5.0, allow_densify=False)
    assert st2 == {"cloned": 0, "split": 0, "pruned": 0}
    assert all(np.array_equal(out2[k], c[k]) for k in NAMES)
