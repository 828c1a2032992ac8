"""CPU restatement of the reference's adaptive density control — TEST
INFRASTRUCTURE ONLY (tests/ use it as the checker; the product never imports it).

Follows gaussian_splatting/utils/adc.py of kmurungi/custom-3dgs-cuda step by
step, in numpy float32, on a cloud given as six arrays (mu [N,3], q [N,4],
s [N,3], alpha [N,1], A [N,3], k_j [N,15,3]) with optional Adam moments:
  stats   (:58-87)    norm of the mean2d gradient scaled by (W/2, H/2) added
                      where > 0, denom + 1 there; max screen radius;
  ADC     (:316-393)  grads = nan_to_num(accum / max(denom, 1));
    clone (:209-240)  grads >= thr and max exp(s) <= percent_dense * extent:
                      the selected appended (moments zero);
    split (:243-294)  on the cloned cloud (grads padded with zeros): grads >=
                      thr and max exp(s) > percent_dense * extent: two copies
                      appended, mu' = R(q) (z * exp(s)) + mu with z the given
                      N(0, 1) rows (the reference's torch.normal draws, copy k of
                      source j in row k n_src + j), s' = log(exp(s) / 1.6); the
                      selected originals dropped; new screen radii 0;
    prune (:373-388)  sigmoid(alpha) < min_opacity, max exp(s) > 0.1 extent,
                      radius > max_screen_size; all pruned -> keep the top
                      max(1, N // 10) by opacity;
    reset (:297-313)  alpha clamped to at most logit(0.01), its moments zero.
Thresholds are fp32 (torch compares an fp32 tensor with a Python float).  exp,
log and sigmoid are numpy's fp32 functions and the rotation product is float32
here; the GPU's differ from these in the last bits (the tests say how much).
"""

from __future__ import annotations

import math

import numpy as np

f32 = np.float32
NAMES = ("mu", "q", "s", "alpha", "A", "k_j")


def stats(accum, denom, maxr, mean2d_grad=None, radii=None, width=None, height=None):
    accum, denom, maxr = (np.array(a, f32, copy=True).reshape(-1) for a in (accum, denom, maxr))
    if mean2d_grad is not None:
        g = np.asarray(mean2d_grad, f32).reshape(-1, 2)[:, :2]
        if width and height and width > 0 and height > 0:
            g = (g * np.array([width / 2.0, height / 2.0], f32)).astype(f32)
        nrm = np.sqrt((g[:, 0] * g[:, 0] + g[:, 1] * g[:, 1]).astype(f32)).astype(f32)
        vis = nrm > 0
        accum[vis] = (accum[vis] + nrm[vis]).astype(f32)
        denom[vis] = (denom[vis] + f32(1.0)).astype(f32)
    if radii is not None:
        r = np.asarray(radii, f32).reshape(-1)
        maxr = np.where(np.isnan(maxr) | np.isnan(r), np.nan, np.maximum(maxr, r)).astype(f32)
    return accum, denom, maxr


def _rotation(q):
    """adc.py:103-119 (F.normalize then the standard matrix), float32."""
    n = np.sqrt((((q[:, 0] * q[:, 0] + q[:, 1] * q[:, 1]) + q[:, 2] * q[:, 2])
                 + q[:, 3] * q[:, 3]).astype(f32)).astype(f32)
    q = (q / np.maximum(n, f32(1e-12))[:, None]).astype(f32)
    w, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    one, two = f32(1), f32(2)
    return np.stack([
        np.stack([one - two * (y * y + z * z), two * (x * y - w * z), two * (x * z + w * y)], -1),
        np.stack([two * (x * y + w * z), one - two * (x * x + z * z), two * (y * z - w * x)], -1),
        np.stack([two * (x * z - w * y), two * (y * z + w * x), one - two * (x * x + y * y)], -1),
    ], 1).astype(f32)


def adc(cloud: dict, moments: dict | None, accum, denom, maxr, noise, *, grad_threshold=0.00005,
        percent_dense=0.01, min_opacity=0.01, max_screen_size=None, scene_extent,
        reset_opacity=False, max_gaussians=800_000, allow_densify=True):
    """(cloud, moments, stats) after the pass.  moments: {name: (exp_avg,
    exp_avg_sq)} or None."""
    c = {k: np.array(cloud[k], f32, copy=True) for k in NAMES}
    m = None if moments is None else {k: [np.array(a, f32, copy=True) for a in moments[k]]
                                      for k in NAMES}
    n0 = c["mu"].shape[0]
    accum = np.asarray(accum, f32).reshape(-1)
    denom = np.asarray(denom, f32).reshape(-1)
    maxr = np.array(maxr, f32, copy=True).reshape(-1)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        den = np.where(np.isnan(denom), denom, np.maximum(denom, f32(1)))
        grads = np.nan_to_num((accum / den).astype(f32), nan=0.0).astype(f32)

    def append(ext: dict, zero_rows: int):
        nonlocal maxr
        for k in NAMES:
            c[k] = np.concatenate([c[k], ext[k]], axis=0)
            if m is not None:
                for j in range(2):
                    m[k][j] = np.concatenate([m[k][j], np.zeros_like(ext[k])], axis=0)
        maxr = np.concatenate([maxr, np.zeros(zero_rows, f32)])

    def keep(mask):
        nonlocal maxr, grads
        for k in NAMES:
            c[k] = c[k][mask]
            if m is not None:
                m[k] = [a[mask] for a in m[k]]
        maxr = maxr[mask]
        grads = grads[mask]

    thr, dense = f32(grad_threshold), f32(percent_dense * scene_extent)
    n_clone = n_split = n_pruned = 0
    with np.errstate(over="ignore"):
        if allow_densify and n0 < max_gaussians:
            smax = np.exp(c["s"]).max(axis=1)
            sel = (grads >= thr) & (smax <= dense)
            n_clone = int(sel.sum())
            if n_clone:
                append({k: c[k][sel] for k in NAMES}, n_clone)
                grads = np.concatenate([grads, np.zeros(n_clone, f32)])
            smax = np.exp(c["s"]).max(axis=1)
            sel = (grads >= thr) & (smax > dense)
            n_split = int(sel.sum())
            if n_split:
                sc = np.exp(c["s"][sel]).astype(f32)
                z = np.asarray(noise, f32).reshape(2 * n_split, 3)
                samples = (z * np.concatenate([sc, sc])).astype(f32)
                rot = np.concatenate([_rotation(c["q"][sel])] * 2)
                new_mu = ((rot[:, :, 0] * samples[:, 0:1] + rot[:, :, 1] * samples[:, 1:2])
                          + rot[:, :, 2] * samples[:, 2:3]).astype(f32)
                new_mu = (new_mu + np.concatenate([c["mu"][sel]] * 2)).astype(f32)
                ext = {k: np.concatenate([c[k][sel]] * 2) for k in NAMES}
                ext["mu"] = new_mu
                ext["s"] = np.log((np.concatenate([sc, sc]) / f32(1.6)).astype(f32)).astype(f32)
                append(ext, 2 * n_split)
                grads = np.concatenate([grads, np.zeros(2 * n_split, f32)])
                keep(~np.concatenate([sel, np.zeros(2 * n_split, bool)]))
        if allow_densify:
            op = (f32(1) / (f32(1) + np.exp(-c["alpha"].reshape(-1)))).astype(f32)
            smax = np.exp(c["s"]).max(axis=1)
            prune = (op < f32(min_opacity)) | (smax > f32(0.1 * scene_extent))
            if max_screen_size is not None:
                prune |= maxr > f32(max_screen_size)
            n = c["mu"].shape[0]
            if prune.any() and (~prune).any():
                n_pruned = int(prune.sum())
                keep(~prune)
            elif n and prune.all():
                k = max(1, n // 10)
                idx = np.argsort(-op, kind="stable")[:k]
                mask = np.zeros(n, bool)
                mask[idx] = True
                n_pruned = n - k
                keep(mask)
            if reset_opacity:
                lv = f32(math.log(0.01 / (1.0 - 0.01)))
                a = c["alpha"]
                c["alpha"] = np.where(np.isnan(a), a, np.minimum(a, lv)).astype(f32)
                if m is not None:
                    m["alpha"] = [np.zeros_like(x) for x in m["alpha"]]
    return c, m, {"cloned": n_clone, "split": n_split, "pruned": n_pruned}
