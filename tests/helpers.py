"""Shared test helpers: run a scene through the CPU oracle, compare arrays."""

from __future__ import annotations

import numpy as np

from oracle import oracle as orc


def scene_arrays(scene) -> dict:
    """numpy copies of a synthetic Scene's parameters and camera (opacity post-sigmoid)."""
    g, v = scene.gaussians, scene.view
    import torch

    f = lambda x: x.detach().cpu().numpy().astype(np.float32)
    R, T = f(v["R"]), f(v["T"])
    return dict(
        mu=f(g.mu), q=f(g.q), s=f(g.s), alpha=f(torch.sigmoid(g.alpha.detach().cpu())),
        A=f(g.A), kj=f(g.k_j), R=R, t=T, cam=(-(R.T @ T)).astype(np.float32).reshape(3),
        fx=float(v["fx"]), fy=float(v["fy"]), cx=float(v["cx"]), cy=float(v["cy"]),
        H=int(v["height"]), W=int(v["width"]))


def oracle_forward(a: dict) -> dict:
    mean2d, cov2d, depth = orc.project(a["mu"], a["q"], a["s"], a["R"], a["t"], a["fx"], a["fy"],
                                       a["cx"], a["cy"])
    colors = orc.sh(a["cam"], a["mu"], a["A"], a["kj"])
    img, ids, ranges, fT, nc, keys = orc.rasterize(depth, mean2d, cov2d, colors, a["alpha"],
                                                   a["H"], a["W"])
    return dict(mean2d=mean2d, cov2d=cov2d, depth=depth, colors=colors, img=img, ids=ids,
                ranges=ranges, final_T=fT, n_contrib=nc, keys=keys)


def bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    return x.view(np.uint32) if x.dtype == np.float32 else x.view(np.uint64)


def assert_bitwise(got, want, what: str) -> None:
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if got.dtype in (np.float32, np.float64):
        same = bits(got) == bits(want)
        # +0 and -0 are the same value; the bar is the value bits otherwise
        same |= (got == 0) & (want == 0)
    else:
        same = got == want
    if not np.all(same):
        idx = np.argwhere(~same)
        first = tuple(idx[0])
        raise AssertionError(
            f"{what}: {idx.shape[0]} of {got.size} elements differ; first at {first}: "
            f"got {got[first]!r} want {want[first]!r}")


def assert_grad_close(got, want, absum, what: str, rel: float = 1e-4,
                      want64=None, floor: float = 0.05,
                      tensor_vs64: bool = False) -> tuple[float, float]:
    """fp32 gradient vs float64 oracle sum.

    Bar: |got - want| <= rel * max(|want|, absum_floor) per element, where the
    floor is rel-scaled by the sum of |terms| (absum) that formed the element:
    an fp32 sum of k terms in any order is accurate to ~k*eps*sum|terms|, so
    elements whose terms cancel are held to the conditioning of their sum, and
    every other element to 1e-4 relative.

    floor: the fraction of absum below which |want| does not shrink the bar
    (0.05: errors up to 5e-6 of sum|terms| pass).  Every term of a pixel's
    gradient scales with its transmittance T, which the backward unwinds from
    final_T through the list; over the ~2000-entry lists of the benchmark scene
    T's relative rounding error at the front of a list reaches ~1e-5 in any
    fp32 evaluation, the reference's own arithmetic included (measured against
    its float64 twin), so those tests pass floor=0.25.

    want64 (optional): the same oracle with float64 per-pixel arithmetic.  The
    fp32 per-pixel arithmetic in the reference's operation order (want) then
    has a measured error of its own on each element, |want - want64|; an
    element also passes when got lies within twice that of want (two fp32
    evaluations of one sum, each with its own rounding).

    Returns (max scaled error over the elements held to the first bar, tensor
    relative error).  The tensor relative error is held to rel against want;
    with tensor_vs64 (needs want64) it is taken against want64 instead and
    held to max(rel, 1.5 x the fp32 oracle's own tensor error against want64):
    over lists of ~1e5 entries per tile the reference's fp32 arithmetic is
    itself a few 1e-4 from float64, and the bar is then to be no less
    accurate than it.
    """
    got = np.asarray(got, dtype=np.float64).reshape(np.shape(want))
    want = np.asarray(want, dtype=np.float64)
    absum = np.asarray(absum, dtype=np.float64).reshape(want.shape)
    scale = np.maximum(np.abs(want), floor * absum)
    scale = np.maximum(scale, 1e-30)
    diff = np.abs(got - want)
    err = diff / scale
    if want64 is not None:
        own = np.abs(want - np.asarray(want64, dtype=np.float64).reshape(want.shape))
        err = np.where(diff <= 2.0 * own, 0.0, err)
    worst = np.unravel_index(np.argmax(err), err.shape) if err.size else None
    assert err.size == 0 or err.max() <= rel, (
        f"{what}: max scaled error {err.max():.3e} > {rel} at {worst}: got {got[worst]!r} "
        f"want {want[worst]!r} absum {absum[worst]!r}"
        + (f" want64 {np.asarray(want64).reshape(want.shape)[worst]!r}" if want64 is not None
           else ""))
    # tensor-level relative error, the plain 1e-4 rel bar
    tot = 0.0
    if tensor_vs64:
        w64 = np.asarray(want64, dtype=np.float64).reshape(want.shape)
        den = np.linalg.norm(w64.ravel())
        if den > 0:
            tot = float(np.linalg.norm((got - w64).ravel()) / den)
            own = float(np.linalg.norm((want - w64).ravel()) / den)
            bar = max(rel, 1.5 * own)
            assert tot <= bar, (f"{what}: tensor relative error against float64 {tot:.3e} > "
                                f"{bar:.3e} (fp32 oracle's own {own:.3e})")
        return (float(err.max()) if err.size else 0.0), tot
    den = np.linalg.norm(want.ravel())
    if den > 0:
        tot = float(np.linalg.norm((got - want).ravel()) / den)
        assert tot <= rel, f"{what}: tensor relative error {tot:.3e} > {rel}"
    return (float(err.max()) if err.size else 0.0), tot


PARAMS = ("mu", "q", "s", "alpha", "A", "k_j")


def rel_error(x, ref) -> float:
    den = np.linalg.norm(ref.ravel())
    return float(np.linalg.norm((x - ref).ravel()) / den) if den > 0 else 0.0


def oracle_chain(a: dict, G, want: dict) -> dict:
    """The six parameter gradients of dL/dimage G through the oracle chain
    (blend backward, SH backward, projection backward, sigmoid backward) on the
    oracle's fp32 forward ``want``, evaluated in float32 and in float64:
    {np.float32: {name: array}, np.float64: {...}}."""
    H, W = a["H"], a["W"]
    chains = {}
    for dt in (np.float32, np.float64):
        dm, dc, dcol, dal = orc.blend_bwd(G, want["mean2d"], want["cov2d"], want["colors"],
                                          a["alpha"], want["ids"], want["ranges"],
                                          want["final_T"], want["n_contrib"], H, W, dtype=dt)
        dA, dkj, dmu_sh = orc.sh_bwd(dcol.astype(dt), a["mu"], a["A"], a["kj"], a["cam"], dtype=dt)
        dmu_p, dq, ds = orc.project_bwd(dm.astype(dt), dc.astype(dt), a["mu"], a["q"], a["s"],
                                        a["R"], a["t"], a["fx"], a["fy"], a["cx"], a["cy"], dtype=dt)
        sig = a["alpha"].astype(np.float64)
        chains[dt] = {"mu": dmu_p.astype(np.float64) + dmu_sh, "q": dq, "s": ds,
                      "alpha": np.asarray(dal, np.float64) * sig * (1.0 - sig), "A": dA, "k_j": dkj}
    return chains


def chain_failures(grads: dict, chains: dict, tag: str) -> list[str]:
    """GPU parameter gradients (name -> float array) against the oracle chain:
    each tensor's relative error to the float64 chain within max(1e-4, 1.5x the
    fp32 chain's own), each element within 1e-4 of the tensor's largest element
    or within twice the fp32 chain's own error on it (a tensor that is zero in
    exact arithmetic, whose fp32 chain is all rounding noise, within twice the
    fp32 chain's largest error).  Prints each tensor's figures; returns the
    failures."""
    fails = []
    for name in PARAMS:
        got = np.asarray(grads[name], np.float64)
        w64 = np.asarray(chains[np.float64][name], np.float64).reshape(got.shape)
        w32 = np.asarray(chains[np.float32][name], np.float64).reshape(got.shape)
        tot, own = rel_error(got, w64), rel_error(w32, w64)
        diff, own_el = np.abs(got - w64), np.abs(w32 - w64)
        top = np.abs(w64).max()
        if own > 1.0:
            bar = np.full(diff.shape, 2.0 * own_el.max())
        else:
            bar = np.maximum(1e-4 * top, 2.0 * own_el)
        bad = diff > bar
        print(f"[gpu] {tag} d_{name}: tensor relative error {tot:.2e} (fp32 chain {own:.2e}); "
              f"max |x| {top:.2e}, max |got - fp64| {diff.max():.2e} (fp32 chain "
              f"{own_el.max():.2e}), elements beyond the bar: {int(bad.sum())}", flush=True)
        fails += [f"{tag} d_{name}: tensor {tot:.3e}"] if tot > max(1e-4, 1.5 * own) else []
        fails += [f"{tag} d_{name}: {int(bad.sum())} elements"] if bad.any() else []
    return fails
