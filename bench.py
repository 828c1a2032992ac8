"""Benchmark of the MI355X rasterizer: fwd+bwd ms/frame and FPS, 100k Gaussians at
1920x1080, with the dominant kernel's HBM-roofline fraction and a CPU baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--no-scale]

A step is one frame of the reference's own benchmark (scripts/bench.py:30-109):
``image = rasterize(gaussians, view)`` then ``image.sum().backward()`` on its synthetic
100k-Gaussian cloud (SH degree-3 coefficients, seed 0) at 1920x1080, inputs resident
in HBM.  Prints one JSON line.  One GPU only: --gpus above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "custom-3dgs-cuda_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fwd+bwd ms/frame & FPS, 100k Gaussians @1920x1080; % HBM roofline"
# Published reference figure on this exact scene (README.md:51, RTX 2060 SUPER):
# 17.724 ms forward + 154.640 ms backward.
REF_FWD_BWD_MS_1080P = 17.724 + 154.640
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, public spec


def _tiles(W, H):
    return ((W + 15) // 16) * ((H + 15) // 16)


def stage_bytes(stage: str, N: int, M: int, W: int, H: int) -> float:
    """Algorithmic bytes per call: the rasterizer baseline's per-stage formulas
    (N Gaussians, M pairs, P pixels, T tiles) for the blends and the per-Gaussian
    stages; the sorts and the schedules use this build's own algorithm."""
    P, T = W * H, _tiles(W, H)
    tile_passes = max(1, math.ceil((T - 1).bit_length() / 8)) if T > 1 else 1
    return {
        "project": 64 * N,
        "sh": 216 * N,
        # one pass: mu, q, s, albedo, k_j in (mu once); mean, cov, depth, radius, colour out
        "project_sh": 272 * N,
        "bin_count": 20 * N + 28 * N,          # mean2d + cov2d + depth in; count, rect, key, val out
        "depth_sort": 4 * 16 * N,
        "scan": 12 * N,
        "records": 36 * N + 48 * N,
        # the first pass generates its pairs from per-Gaussian data (perm,
        # offset, rect: 16 B) and writes 8 B per pair; later passes move 16 B
        "tile_sort": (16 * tile_passes - 8) * M + 16 * N,
        "ranges": 4 * M + 8 * T,
        # depth order + rects read twice per level-1 pass, block lists written
        # once and read twice (counted at one entry per Gaussian), ids written
        "tile_binning": 4 * M + 2 * 12 * N + 3 * 4 * N + 8 * T,
        "fwd_schedule": 16 * T,                 # ranges in, estimates + order out (walk not counted)
        "blend_fwd": 40 * M + 20 * P + 8 * T,
        # mean2d, cov2d, colour, opacity in; record, count, rect, slot offset out
        "bwd_records": 100 * N,
        "bwd_schedule": 4 * P + 16 * T,
        "blend_bwd": 76 * M + 20 * P + 8 * T,
        "grad_reduce": M // 8 + 8 * N,          # slot flag bits + offsets (sums of processed pairs not counted)
        "sh_bwd": 420 * N,
        "project_bwd": 100 * N,
        # the two backwards in one pass: mu read once, dL/dmu written once
        "project_sh_bwd": 496 * N,
        # the trainer's loss: both images in, the SSIM index's three derivative
        # maps out (fwd); maps and images in, dL/dimage out (bwd)
        "loss": 60 * P,
        "loss_bwd": 72 * P,
        # the fused optimizer step over the 59 fp32 parameters of a Gaussian:
        # parameter, gradient and both moments in, parameter and moments out
        "adam": 28 * 59 * N,
        # the PLY export's records: 59 parameters in, 62-float records out
        "ply_pack": 236 * N + 248 * N,
        # densification statistics: mean2d gradient and radius in, the three
        # buffers read and written
        "adc_stats": 12 * N + 24 * N,
        # the densify / prune plan: buffers, log-scales and opacity in, flags out
        "adc_plan": 29 * N,
        # the gather: every parameter and both moments read and written once
        # (counted for a pass that keeps each Gaussian once)
        "adc_apply": 2 * 3 * 236 * N,
    }.get(stage)


# VALU issue ceiling from MI355X's published figures: 256 CUs x 4 SIMDs, each
# SIMD issuing one wave64 VALU instruction per 4-cycle quad-cycle, at the
# 2.4 GHz peak engine clock: 614.4 G issue quad-cycles/s.  The same figure is
# the published 157.3 TFLOP/s fp32 vector peak divided by the 256 flops of a
# wave64 packed FMA.  Two VALU instructions can share a quad-cycle (rocprofv3's
# SQ_ACTIVE_INST_VALU2), so a kernel's issue quad-cycles are SQ_ACTIVE_INST_VALU
# - SQ_ACTIVE_INST_VALU2 (transcendentals and lane permutes take two).
VALU_PEAK_GISSUE = 256 * 4 * 2.4 / 4
# The blends are bound by VALU issue, not by HBM: their pct_hbm_peak comes only
# from measured FETCH_SIZE + WRITE_SIZE traffic, never from a byte formula.
VALU_BOUND_STAGES = ("blend_fwd", "blend_bwd")
# Calibration kinds of gsr_calibrate_valu (one instruction kind per kernel).
VALU_CALIBRATION_KINDS = ("add", "fma", "exp", "permlane_swap", "dpp_add")


def _profile_json(kind: str, workload: str):
    """profiles/<kind>_<workload>.json (committed summaries of rocprofv3 runs)."""
    p = ROOT / "profiles" / f"{kind}_{workload}.json"
    if p.exists():
        try:
            return json.loads(p.read_text())
        except (OSError, ValueError):
            return None
    return None


# Sources whose change can change any stage's kernels: the shared device headers
# and the host code that sizes the workspaces and sets the launch order.
SHARED_SOURCES = ("gsr_common.h", "gsr_math.h", "gsr_gaussian.h", "gsr_group.h",
                  "gsr_internal.h", "gsr_schedule.h", "gsr_capi.cpp")


def library_sources() -> dict:
    """{file: sha256 prefix} of the sources the loaded libgsraster.so was built
    from (gsr_build_sources)."""
    import custom_rasterizer_cuda as crc

    return dict(item.split("=", 1) for item in crc.library_sources().split(";") if "=" in item)


def stale_reason(profile, entry) -> str | None:
    """None when the kernels a profile entry measured are built from the same
    sources as the loaded library: every file in the entry's "source_files"
    plus SHARED_SOURCES has the hash the profile's "sources" recorded.
    Otherwise the reason its counters no longer describe this build."""
    if not profile or not entry:
        return "no profile entry"
    rec = profile.get("sources")
    if not rec:
        return "the profile records no source hashes"
    cur = library_sources()
    if not cur:
        return "the loaded library records no source hashes"
    files = sorted(set(entry.get("source_files") or cur) | set(SHARED_SOURCES))
    changed = [f for f in files if rec.get(f) != cur.get(f)]
    if changed:
        return "sources changed since the profile: " + ", ".join(changed)
    return None


def dominant_roofline(stage: str, per_stage: dict, N: int, M: int, W: int, H: int,
                      workload: str) -> dict:
    """The roofline object of the frame's dominant stage, its average launch
    time measured live (HIP events around each launch on the launch stream).

    VALU-bound blends: achieved = the kernel's VALU issue quad-cycles per launch
    (SQ_ACTIVE_INST_VALU - SQ_ACTIVE_INST_VALU2, profiles/valu_<workload>.json)
    / launch time, against VALU_PEAK_GISSUE; the issue utilisation at the
    measured clock and the calibration kernels' utilisation (the practical
    ceiling of one instruction kind) come from the same profile.  The HBM side
    is the measured FETCH_SIZE + WRITE_SIZE traffic; the per-pair byte formula
    is kept as a labelled equivalent.  Other stages: HBM-bound, achieved =
    their formula bytes / launch time."""
    avg_s = per_stage[stage]["ms"] * 1e-3
    alg = stage_bytes(stage, N, M, W, H)
    tp = _profile_json("traffic", workload)
    tr = (tp or {}).get("stages", {}).get(stage)
    tr_stale = stale_reason(tp, tr)
    traffic = tr.get("bytes_per_call") if tr and not tr_stale else None
    va = (_profile_json("valu", workload) or {})
    vk = va.get("kernels", {}).get(stage)
    va_stale = stale_reason(va, vk)
    if stage in VALU_BOUND_STAGES and va_stale:
        # the issue counts were measured on other kernel code: no fraction
        return {"bound": "valu", "kernel": stage, "achieved": None, "peak": VALU_PEAK_GISSUE,
                "unit": "G VALU issue quad-cycles/s", "frac": None, "traffic": traffic,
                "avg_launch_ms": per_stage[stage]["ms"],
                "reason": "VALU counters: " + va_stale
                + ("" if not tr_stale else "; HBM counters: " + tr_stale)}
    if stage in VALU_BOUND_STAGES and vk:
        ach = vk["issue_quads_per_launch"] / avg_s / 1e9
        out = {"bound": "valu", "kernel": stage, "achieved": round(ach, 1),
               "peak": VALU_PEAK_GISSUE, "unit": "G VALU issue quad-cycles/s",
               "frac": round(ach / VALU_PEAK_GISSUE, 4), "traffic": traffic,
               "avg_launch_ms": per_stage[stage]["ms"],
               "issue_quads_per_launch": vk["issue_quads_per_launch"],
               "valu_insts_per_launch": vk.get("insts_per_launch"),
               "issue_util_at_measured_clock": vk.get("issue_util"),
               "measured_clock_mhz": vk.get("clock_mhz"),
               "calibration_issue_util": {k: c.get("issue_util")
                                          for k, c in va.get("calibration", {}).items()}}
        if traffic:
            gbs = traffic / avg_s / 1e9
            out["hbm_measured"] = {"GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        if alg:
            gbs = alg / avg_s / 1e9
            out["equivalent"] = {"what": "the rasterizer baseline's per-pair byte formula",
                                 "bytes": alg, "GBps": round(gbs, 1),
                                 "frac": round(gbs / HBM_PEAK_GBS, 4)}
        return out
    b = traffic or alg
    ach = (b / avg_s / 1e9) if b else 0.0
    out = {"bound": "hbm", "kernel": stage, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
           "algorithmic_bytes": alg, "avg_launch_ms": per_stage[stage]["ms"]}
    if tr and tr_stale:
        out["traffic_note"] = "measured traffic not used: " + tr_stale
    return out


def _clear(g):
    for name in ("mu", "q", "s", "alpha", "A", "k_j"):
        getattr(g, name).grad = None


# The reference's scripts/bench.py runs 100 untimed iterations before it times
# (its --warmup default, scripts/bench.py:124-127), so its published figure is
# a warm GPU's.  The headline frame is timed after the same 100 untimed frames,
# continued until they have run for at least REF_WARMUP_S (reported as
# "reference_warmup"), then the command line's W warmup steps and K timed
# steps.  An idle MI355X takes tens of milliseconds of load to reach its
# clocks: 20 timed frames after 5 warmup steps measured 0.597 ms per frame,
# after 100 0.562 ms, and 200 after 20 0.561 ms.
REF_WARMUP_FRAMES = 100
REF_WARMUP_S = 0.25


def time_frames(sc, steps: int, warmup: int, profile: bool, render=None, grad=None,
                prewarm: int = 0):
    """Mean forward, backward and whole-frame ms of ``steps`` frames, after
    ``prewarm`` + ``warmup`` untimed ones.  The backward is
    ``image.sum().backward()`` (the reference's bench.py:94-96), or
    ``image.backward(grad)`` for a given dL/dimage (the baseline configs'
    seeded N(0, 1))."""
    import torch
    import custom_rasterizer_cuda as crc
    from gaussian_splatting.rasterizer.rasterize import rasterize

    rasterize = render or rasterize
    g, view = sc.gaussians, sc.view

    def backward(img):
        if grad is None:
            img.sum().backward()
        else:
            img.backward(grad)

    t0, done = time.perf_counter(), 0
    while prewarm and (done < prewarm or time.perf_counter() - t0 < REF_WARMUP_S):
        _clear(g)
        backward(rasterize(g, view))
        done += 1
        if done % 20 == 0:
            torch.cuda.synchronize()
    for _ in range(warmup):
        _clear(g)
        backward(rasterize(g, view))
    torch.cuda.synchronize()
    crc.profile_reset()
    crc.profile_enable(profile)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for e0, e1, e2 in ev:
        _clear(g)
        e0.record()
        img = rasterize(g, view)
        e1.record()
        backward(img)
        e2.record()
    t_end.record()
    torch.cuda.synchronize()
    crc.profile_enable(False)
    stages = crc.profile_collect() if profile else {}
    fwd = sum(a.elapsed_time(b) for a, b, _ in ev) / steps
    bwd = sum(b.elapsed_time(c) for _, b, c in ev) / steps
    total = t_start.elapsed_time(t_end) / steps
    return fwd, bwd, total, stages


def pair_count(sc) -> int:
    import torch
    import custom_rasterizer_cuda as crc

    g, v = sc.gaussians, sc.view
    with torch.no_grad():
        n = g.mu.shape[0]
        m2, c2, d = crc.project(n, g.mu.detach(), g.q.detach(), g.s.detach(), v["R"], v["T"],
                                float(v["fx"]), float(v["fy"]), float(v["cx"]), float(v["cy"]))
        cam = -(v["R"].T @ v["T"])
        col = crc.SH(n, cam.contiguous(), g.mu.detach(), g.A.detach(), g.k_j.detach())
        out = crc.rasterize(n, d, m2, c2, col, torch.sigmoid(g.alpha.detach()), v["height"],
                            v["width"])
    return int(out[1].numel())


def _stage_rates(stages: dict, N: int, M: int, W: int, H: int, keep=None,
                 workload: str | None = None) -> dict:
    """Per-stage ms and HBM rate.  The bytes are the stage's measured
    FETCH_SIZE + WRITE_SIZE per call where profiles/traffic_<workload>.json
    holds them ("bytes": "measured"), else the per-stage formula
    ("bytes": "formula"); the VALU-bound blends get no formula rate."""
    prof = _profile_json("traffic", workload) if workload else None
    measured = (prof or {}).get("stages", {})
    out = {}
    for name, (count, ms) in stages.items():
        if keep is not None and name not in keep:
            continue
        avg = ms / max(count, 1)
        entry = {"ms": round(avg, 4), "calls": int(count)}
        b, src = None, None
        stale = stale_reason(prof, measured.get(name)) if name in measured else None
        if name in measured and measured[name].get("bytes_per_call") and not stale:
            b, src = float(measured[name]["bytes_per_call"]), "measured"
        elif name not in VALU_BOUND_STAGES:
            b, src = stage_bytes(name, N, M, W, H), "formula"
        if stale:
            entry["measured_bytes_not_used"] = stale
        if b is not None and avg > 0:
            gbs = b / (avg * 1e-3) / 1e9
            entry.update({"GBps": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                          "bytes": src})
        else:
            entry.update({"GBps": None, "pct_hbm_peak": None, "bytes": None})
        if name in VALU_BOUND_STAGES:
            entry["bound"] = "valu"
        out[name] = entry
    return out


# The stages that replace the reference's count_overlaps + exclusive scan +
# key_generation + 64-bit radix sort + tile ranges (rasterize.cu:345-449).
BINNING_STAGES = ("bin_count", "depth_sort", "scan", "tile_binning", "tile_sort", "ranges")


def reference_binning_bytes(N: int, M: int, W: int, H: int) -> int:
    """The rasterizer baseline's fixed algorithmic bytes for those stages: count +
    scan + keys 64N + 12M, the sort's passes x 24M with passes = ceil((32 +
    ceil(log2 T)) / 8) 8-bit digits, ranges 8M + 8T."""
    T = _tiles(W, H)
    passes = math.ceil((32 + math.ceil(math.log2(T)) if T > 1 else 32) / 8)
    return 64 * N + 12 * M + passes * 24 * M + 8 * M + 8 * T


def binning_summary(stages: dict, N: int, M: int, W: int, H: int) -> dict:
    """Time of the binning stages against the reference algorithm's bytes (an
    equivalent rate: this build moves fewer bytes) and against this build's own."""
    used = [k for k in BINNING_STAGES if k in stages]
    ms = sum(stages[k]["ms"] for k in used)
    own = sum(stage_bytes(k, N, M, W, H) for k in used)
    ref = reference_binning_bytes(N, M, W, H)
    if ms <= 0:
        return {"stages": used, "ms": 0.0}
    return {"stages": used, "ms": round(ms, 4), "reference_bytes": ref,
            "reference_equiv_GBps": round(ref / (ms * 1e-3) / 1e9, 1),
            "reference_equiv_frac": round(ref / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3),
            "own_bytes": own, "own_GBps": round(own / (ms * 1e-3) / 1e9, 1),
            "own_frac": round(own / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}


def per_gaussian_stages(sc, calls: int = 20) -> dict:
    """The per-Gaussian stages (project, SH, their backwards and the fused glue
    kernels) called directly on config ``sc``'s cloud, at sizes where they move
    hundreds of MB: HIP-event stage times and GB/s from the per-stage byte
    formulas."""
    import torch
    import custom_rasterizer_cuda as crc

    g, v = sc.gaussians, sc.view
    n = g.mu.shape[0]
    mu, q, s, A, kj = (x.detach() for x in (g.mu, g.q, g.s, g.A, g.k_j))
    logits = g.alpha.detach()
    R, T = v["R"], v["T"]
    fx, fy, cx, cy = (float(v[k]) for k in ("fx", "fy", "cx", "cy"))
    gen = torch.Generator(device="cpu").manual_seed(7)
    dm = torch.randn(n, 2, generator=gen).to(mu.device)
    dc = torch.randn(n, 3, generator=gen).to(mu.device)
    dcol = torch.randn(n, 3, generator=gen).to(mu.device)
    dal = torch.randn(n, 1, generator=gen).to(mu.device)
    cam = (-(R.T @ T)).contiguous()

    # the optimizer step over the cloud's six parameter tensors (values are
    # arbitrary: the kernel's work does not depend on them)
    params = [x.clone() for x in (mu, q, s, logits, A, kj)]
    grads = [torch.randn_like(x) for x in params]
    moms = [torch.zeros_like(x) for x in params]
    vars_ = [torch.zeros_like(x) for x in params]
    lrs = [1.6e-4, 1e-3, 5e-3, 5e-2, 2.5e-3, 6.25e-4]
    inf = float("inf")

    def one_round():
        crc.adam_step(params, grads, moms, vars_, lrs, [1] * 6, [-inf] * 6, [inf] * 6, 0.9,
                      0.999, 1e-15)
        crc.ply_records(mu, q, s, logits, A, kj, False)
        crc.project(n, mu, q, s, R, T, fx, fy, cx, cy)
        crc.SH(n, cam, mu, A, kj)
        out = crc.project_sh(n, mu, q, s, R, T, fx, fy, cx, cy, A, kj, logits)
        crc.backwards_SH(dcol, mu, A, kj, cam)
        crc.backwards_projection(dm, dc, mu, q, s, R, T, fx, fy, cx, cy)
        crc.backwards_project_sh(dm, dc, dcol, mu, q, s, R, T, fx, fy, A, kj, out[5], dal,
                                 out[6])

    with torch.no_grad():
        for _ in range(3):
            one_round()
        torch.cuda.synchronize()
        crc.profile_reset()
        crc.profile_enable(True)
        for _ in range(calls):
            one_round()
        torch.cuda.synchronize()
        crc.profile_enable(False)
        stages = crc.profile_collect()
    out = _stage_rates(stages, n, 0, v["width"], v["height"])
    # VALU issue beside the HBM rate: the kernels' issue quad-cycles per launch
    # at this size (profiles/valu_per_gaussian_c5_5M.json) over the live time
    # against VALU_PEAK_GISSUE (the projection backward is issue-bound)
    vp = _profile_json("valu", "per_gaussian_c5_5M")
    vk = (vp or {}).get("kernels", {})
    if n == 5_000_000:
        for name, entry in out.items():
            k = vk.get(name)
            stale = stale_reason(vp, k) if k else None
            if stale:
                entry["valu"] = {"kernel": k["kernel"], "frac": None, "reason": stale}
            elif k and entry["ms"] > 0:
                ach = k["issue_quads_per_launch"] / (entry["ms"] * 1e-3) / 1e9
                entry["valu"] = {"kernel": k["kernel"], "G_issue_quads_per_s": round(ach, 1),
                                 "frac": round(ach / VALU_PEAK_GISSUE, 4)}
    return out


def train_steps(sc, steps: int, warmup: int = 3) -> dict:
    """The reference trainer's step (scripts/train.py:148-178) on scene ``sc``:
    rasterize, the L1 + D-SSIM loss against a fixed target image, backward,
    the densification statistics, the fused Adam step with the opacity and
    log-scale clamps; ms per step and the per-stage breakdown."""
    import torch
    import custom_rasterizer_cuda as crc
    from gaussian_splatting.rasterizer.rasterize import rasterize
    from gaussian_splatting.rasterizer.rasterize import RasterizeFunction
    from gaussian_splatting.utils.adc import densification_stats
    from gaussian_splatting.utils.loss import calculate_loss
    from gaussian_splatting.utils.optim import setup_optimizer, set_trainer_clamps

    g, v = sc.gaussians, sc.view
    H, W = int(v["height"]), int(v["width"])
    gen = torch.Generator(device="cpu").manual_seed(11)
    target = torch.rand(H, W, 3, generator=gen).to(g.mu.device)
    lrs = {"mu": 1.6e-4, "q": 1e-3, "s": 5e-3, "alpha": 5e-2, "A": 2.5e-3, "k_j": 6.25e-4}
    opt = setup_optimizer(g, lrs)
    set_trainer_clamps(opt, scene_extent=5.0)

    def step():
        opt.zero_grad(set_to_none=True)
        loss = calculate_loss(target, rasterize(g, v))
        loss.backward()
        densification_stats(g, RasterizeFunction.last_mean2d_grad, RasterizeFunction.last_radii2d,
                            width=W, height=H)
        opt.step()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        step()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    crc.profile_reset()
    crc.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    crc.profile_enable(False)
    stages = crc.profile_collect()
    M = pair_count(sc)
    return {"ms_per_step": round(ms, 4), "steps_per_s": round(1000.0 / ms, 1), "pairs": M,
            "stages": _stage_rates(stages, sc.n, M, W, H)}


def adc_pass(sc, calls: int = 3) -> dict:
    """The densify / prune pass (utils/adc.py:316-393) on config ``sc``'s cloud
    with Adam state, statistics that select about a tenth of the Gaussians
    for densification: ms per pass and the per-stage breakdown (the cloud is
    rebuilt from the same inputs each call)."""
    import torch
    import custom_rasterizer_cuda as crc
    from gaussian_splatting.scene.gaussian import gaussian
    from gaussian_splatting.utils.adc import adaptive_density_control
    from gaussian_splatting.utils.optim import setup_optimizer

    src = sc.gaussians
    n = src.mu.shape[0]
    gen = torch.Generator(device="cpu").manual_seed(5)
    accum = (torch.rand(n, 1, generator=gen) * 1.1e-4).to(src.mu.device)
    lrs = {"mu": 1.6e-4, "q": 1e-3, "s": 5e-3, "alpha": 5e-2, "A": 2.5e-3, "k_j": 6.25e-4}

    def fresh():
        g = gaussian(n)
        for k in ("mu", "q", "s", "alpha", "A", "k_j"):
            setattr(g, k, getattr(src, k).detach().clone())
        opt = setup_optimizer(g, lrs)
        for p in opt.param_groups:
            par = p["params"][0]
            opt.state[par] = {"step": torch.tensor(1.0), "exp_avg": torch.zeros_like(par),
                              "exp_avg_sq": torch.zeros_like(par)}
        g.xyz_grad_accum = accum.clone()
        g.denom = torch.ones_like(accum)
        g.max_radii2D = torch.zeros(n, device=src.mu.device)
        return g, opt

    g, opt = fresh()
    kw = dict(scene_extent=5.0, max_screen_size=200.0, max_gaussians=4 * n)
    adaptive_density_control(g, opt, **kw)
    times, stats = [], None
    crc.profile_reset()
    crc.profile_enable(True)
    for _ in range(calls):
        g, opt = fresh()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g, opt, stats = adaptive_density_control(g, opt, **kw)
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    crc.profile_enable(False)
    stages = crc.profile_collect()
    return {"ms_per_pass": round(sorted(times)[len(times) // 2], 3), "gaussians": n,
            "result": stats, "stages": _stage_rates(stages, n, 0, 0, 0)}


def config_grad(sc):
    """The baseline configs' dL/dimage: N(0, 1), seeded, resident on the device."""
    from gaussian_splatting import synthetic

    v = sc.view
    return synthetic.grad_image(int(v["height"]), int(v["width"]), seed=3).to(
        sc.gaussians.mu.device)


def frame_stages(sc, steps: int, binning: str | None = None) -> dict:
    """fwd+bwd frames of config ``sc`` (dL/dimage N(0, 1)) with the per-stage
    breakdown; ``binning`` "sort" selects the LSD tile sort (GSR_TILE_BINNING)
    for these frames."""
    old = os.environ.get("GSR_TILE_BINNING")
    if binning:
        os.environ["GSR_TILE_BINNING"] = binning
    try:
        M = pair_count(sc)
        G = config_grad(sc)
        fwd, bwd, total, _ = time_frames(sc, steps, 2, profile=False, grad=G)
        _, _, _, stages = time_frames(sc, steps, 1, profile=True, grad=G)
    finally:
        if old is None:
            os.environ.pop("GSR_TILE_BINNING", None)
        else:
            os.environ["GSR_TILE_BINNING"] = old
    v = sc.view
    rates = _stage_rates(stages, sc.n, M, v["width"], v["height"],
                         workload=sc.name + "_randn_grad" + (f"_tile_{binning}" if binning else ""))
    return {"fwd_ms": round(fwd, 4), "bwd_ms": round(bwd, 4), "ms_per_frame": round(total, 4),
            "fps": round(1000.0 / total, 1), "pairs": M,
            "binning": binning_summary(rates, sc.n, M, v["width"], v["height"]),
            "stages": rates}


def band_plan(sc, band_height: int | None):
    """The bands rasterize_bands renders config ``sc``'s frame in, and each
    band's pair count (the frame's pairs per tile row summed over the band)."""
    import torch
    import custom_rasterizer_cuda as crc
    from gaussian_splatting.rasterizer.bands import band_rows, plan_bands

    g, v = sc.gaussians, sc.view
    H, W = int(v["height"]), int(v["width"])
    with torch.no_grad():
        n = g.mu.shape[0]
        m2, c2, _ = crc.project(n, g.mu.detach(), g.q.detach(), g.s.detach(), v["R"], v["T"],
                                float(v["fx"]), float(v["fy"]), float(v["cx"]), float(v["cy"]))
        rows = crc.tile_row_pairs(n, m2, c2, H, W).cpu().tolist()
    plan = plan_bands(rows, H) if band_height is None else band_rows(H, band_height)
    return plan, [sum(rows[y0 // 16:(y0 + h + 15) // 16]) for y0, h in plan]


def banded_frame(sc, band_height: int | None, steps: int) -> dict:
    """fwd+bwd of a frame beyond the int32 pair lists, rendered as screen bands
    through the unchanged surface (rasterize_bands): bands planned from the
    frame's pairs per tile row (band_height None) or of ``band_height`` rows;
    frame time, the stage breakdown and each band's pair count."""
    import torch
    from gaussian_splatting.rasterizer.bands import rasterize_bands

    render = lambda g, v: rasterize_bands(g, v, band_height)
    plan, pairs = band_plan(sc, band_height)
    print(f"[bench] {sc.name}: {steps} banded frame(s), {len(plan)} bands "
          f"({'planned' if band_height is None else f'{band_height} rows'})",
          file=sys.stderr, flush=True)
    G = config_grad(sc)
    fwd, bwd, total, _ = time_frames(sc, steps, 1, profile=False, render=render, grad=G)
    _, _, _, stages = time_frames(sc, 1, 0, profile=True, render=render, grad=G)
    from gaussian_splatting.rasterizer import bands as bands_mod
    prefix_stats = bands_mod.prefix_stats()
    print(f"[bench] {sc.name}: {total:.1f} ms per frame ({prefix_stats})", file=sys.stderr,
          flush=True)
    torch.cuda.empty_cache()
    v = sc.view
    rates = {}
    for name, (count, ms) in stages.items():  # one profiled frame
        rates[name] = {"ms_per_frame": round(ms, 3), "calls": int(count)}
    return {"fwd_ms": round(fwd, 3), "bwd_ms": round(bwd, 3), "ms_per_frame": round(total, 3),
            "fps": round(1000.0 / total, 2), "pairs": sum(pairs), "bands": len(plan),
            "band_rows": [h for _, h in plan], "band_pairs": pairs,
            "band_plan": "pairs per tile row, at most (2^31 - 2^16) x 127/128 per band"
            if band_height is None else f"{band_height} rows",
            "max_band_pairs": max(pairs),
            # what the frames rendered: depth-prefix rendering's two passes
            # (prefix, pairs and bands of each) or the planned bands
            "rendered": prefix_stats,
            "stages": rates, "width": v["width"], "height": v["height"], "gaussians": sc.n}


def cpu_baseline(sc, budget_s: float = 30.0) -> dict:
    """The CPU oracle (oracle/gs_oracle.cpp, OpenMP) on the same frame: forward
    (project, SH, key emission, stable sort, ranges, blend) + backward (blend, SH,
    projection) with dL/dimg = 1 (image.sum())."""
    import numpy as np
    import torch
    from oracle import oracle as orc

    # Every core the process may run on, up to the host's share for one GPU
    # (GSR_CPU_SHARE, default 16: the GPU pool's boxes give one GPU's job 16 of
    # their cores, whatever the machine has in all).
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (
        os.cpu_count() or 1)
    share = int(os.environ.get("GSR_CPU_SHARE", "16"))
    threads = max(1, min(avail, share) if share > 0 else avail)
    g, v = sc.gaussians, sc.view
    f = lambda t: t.detach().cpu().numpy().astype(np.float32)
    mu, q, s, A, kj = f(g.mu), f(g.q), f(g.s), f(g.A), f(g.k_j)
    op = f(torch.sigmoid(g.alpha.detach().cpu()))
    R, T = f(v["R"]), f(v["T"])
    H, W = v["height"], v["width"]
    cam = (-(R.T @ T)).astype(np.float32)
    G = np.ones((H, W, 3), np.float32)
    pairs = 0

    def frame():
        nonlocal pairs
        t0 = time.perf_counter()
        m2, c2, d = orc.project(mu, q, s, R, T, v["fx"], v["fy"], v["cx"], v["cy"])
        col = orc.sh(cam, mu, A, kj)
        img, ids, ranges, fT, nc, _ = orc.rasterize(d, m2, c2, col, op, H, W)
        dm, dc, dcol, dop = orc.blend_bwd(G, m2, c2, col, op, ids, ranges, fT, nc, H, W)
        dA, dkj, dmu_sh = orc.sh_bwd(dcol.astype(np.float32), mu, A, kj, cam)
        orc.project_bwd(dm.astype(np.float32), dc.astype(np.float32), mu, q, s, R, T, v["fx"],
                        v["fy"], v["cx"], v["cy"])
        pairs = ids.size
        return time.perf_counter() - t0

    # the median of three frames on `threads` threads, then one single-threaded
    # frame if the budget has room for it (about 16x the threaded time)
    orc.set_threads(threads)
    times = []
    t_begin = time.perf_counter()
    while True:
        times.append(frame())
        if time.perf_counter() - t_begin + times[-1] > budget_s or len(times) >= 3:
            break
    ms = 1000.0 * sorted(times)[len(times) // 2]
    one = None
    if threads > 1 and time.perf_counter() - t_begin + threads * ms * 1e-3 <= budget_s:
        orc.set_threads(1)
        one = round(1000.0 * frame(), 1)
        orc.set_threads(threads)
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")),
                         None)
    except OSError:
        pass
    return {"value": round(1000.0 / ms, 4), "unit": "frames/s", "cores": threads, "kind": "port",
            "ms_per_frame": round(ms, 1), "ms_per_frame_1_thread": one,
            "nproc": os.cpu_count(), "cores_available": avail, "cpu_share": share,
            "cpu_model": model,
            "sample": f"median of {len(times)} full frame(s) fwd+bwd of the same workload "
                      f"({g.mu.shape[0]} Gaussians, {W}x{H}, {pairs} pairs) through the "
                      f"fp32 CPU oracle with {threads} OpenMP threads"
                      + (", and one frame on 1 thread" if one is not None else "")}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--gaussians", type=int, default=100_000)
    ap.add_argument("--width", type=int, default=1920)
    ap.add_argument("--height", type=int, default=1080)
    ap.add_argument("--scene", default="bench", choices=["bench", "c1", "c2", "c3", "c4", "c5"],
                    help="the frame to time: the reference's bench scene (default) or a "
                         "rasterizer baseline config at its own size (for profiling)")
    ap.add_argument("--grad", default="sum", choices=["sum", "randn"],
                    help="dL/dimage of the timed frames: image.sum() (the reference's "
                         "bench.py, default) or the baseline configs' seeded N(0, 1)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-c5", action="store_true",
                    help="skip config c5 (5M Gaussians, 3840x2160, timed in screen bands)")
    ap.add_argument("--band-height", type=int, default=0,
                    help="rows per screen band of the c5 frame (a multiple of 16); 0 (default): "
                         "bands planned from the frame's pairs per tile row")
    ap.add_argument("--no-extra", action="store_true", help="skip the 720p and c3 side runs")
    ap.add_argument("--no-scale", action="store_true",
                    help="skip the per-stage HBM measurements on configs c4 and c5")
    ap.add_argument("--calibrate-valu", action="store_true",
                    help="only run the VALU issue-rate calibration kernels (one per "
                         "instruction kind, 3 launches each) and print their rates")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the rasterizer path here runs on a single MI355X "
              "(multi-GPU screen-band sharding is a design note, not built). Use --gpus 1.",
              file=sys.stderr)
        return 2

    import torch
    from gaussian_splatting import synthetic

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda")
    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4,
                          "launches": 5}), flush=True)
        return 0
    if args.calibrate_valu:
        import custom_rasterizer_cuda as crc

        iters, res = 4096, {}
        for kind, name in enumerate(VALU_CALIBRATION_KINDS):
            best = None
            for _ in range(3):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                out = crc.calibrate_valu(kind, iters)
                b.record()
                torch.cuda.synchronize()
                ms = a.elapsed_time(b)
                best = ms if best is None else min(best, ms)
            insts = out.numel() // 64 * iters * 8  # wave64 instructions of the kind
            res[name] = {"ms": round(best, 4), "wave64_insts": insts,
                         "G_insts_per_s": round(insts / (best * 1e-3) / 1e9, 1)}
        print(json.dumps({"calibrate_valu": res}), flush=True)
        return 0
    W, H, N = args.width, args.height, args.gaussians
    if args.scene == "bench":
        sc = synthetic.bench_scene(n=N, width=W, height=H, device=dev)
        workload = f"bench_{N // 1000}k_{W}x{H}"
    else:
        sc = synthetic.config_scene(args.scene, device=dev)
        N, W, H = sc.n, sc.view["width"], sc.view["height"]
        workload = sc.name
    M = pair_count(sc)

    G = config_grad(sc) if args.grad == "randn" else None
    if G is not None:
        workload += "_randn_grad"
    fwd, bwd, total, _ = time_frames(sc, args.steps, args.warmup, profile=False, grad=G,
                                     prewarm=REF_WARMUP_FRAMES)
    pf, pb, ptot, stages = time_frames(sc, args.steps, 2, profile=True, grad=G)

    per_stage = _stage_rates(stages, N, M, W, H, workload=workload)
    dominant = max(per_stage, key=lambda k: per_stage[k]["ms"]) if per_stage else None
    roofline = dominant_roofline(dominant, per_stage, N, M, W, H, workload) if dominant else None

    value = 1000.0 / total
    out = {
        "metric": METRIC, "value": round(value, 3), "unit": "frames/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total, 4),
        # untimed frames before the warmup steps: the reference's own protocol
        "reference_warmup": {"frames": REF_WARMUP_FRAMES, "min_s": REF_WARMUP_S},
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(value / (1000.0 / REF_FWD_BWD_MS_1080P), 2)
        if (W, H, N) == (1920, 1080, 100_000) else None,
        "dtype": "fp32", "data": "synthetic",
        "config": {"workload": (f"reference scripts/bench.py scene, {N} Gaussians (SH-3 "
                                f"coefficients, seed 0), {W}x{H}, forward + backward "
                                f"(loss = image.sum())") if args.scene == "bench" else
                               f"rasterizer baseline config {sc.name}, forward + backward "
                               f"(loss = {'image.sum()' if G is None else 'dL/dimage N(0,1)'})",
                   "gaussians": N, "width": W, "height": H, "pairs": M, "tiles": _tiles(W, H)},
        "fwd_ms": round(fwd, 4), "bwd_ms": round(bwd, 4),
        "fps_forward": round(1000.0 / fwd, 1),
        "roofline": roofline,
        "binning": binning_summary(per_stage, N, M, W, H),
        "stages": per_stage,
        "profiled_ms_per_step": round(ptot, 4),
        # the sha256 prefixes of the sources the measured library was built from
        "build_sources": library_sources(),
    }
    if not args.no_extra:
        extra = {}
        # the 720p bench scene (image.sum(), as the reference's bench.py), the
        # 1080p bench scene with a seeded N(0, 1) dL/dimage, and configs c2 and
        # c3 (N(0, 1) dL/dimage, as the baseline states)
        b1080 = synthetic.bench_scene(n=N, width=1920, height=1080, device=dev)
        for label, scene, grad in (
                ("bench_100k_1280x720",
                 synthetic.bench_scene(n=N, width=1280, height=720, device=dev), None),
                ("bench_100k_1920x1080_randn_grad", b1080, config_grad(b1080)),
                ("c2_100k_1280x720", synthetic.config_scene("c2", device=dev), "randn"),
                ("c3_100k_1920x1080", synthetic.config_scene("c3", device=dev), "randn")):
            if isinstance(grad, str):
                grad = config_grad(scene)
            f2, b2, t2, _ = time_frames(scene, max(10, args.steps // 2), 5, profile=False,
                                        grad=grad)
            extra[label] = {"fwd_ms": round(f2, 4), "bwd_ms": round(b2, 4),
                            "ms_per_frame": round(t2, 4), "fps": round(1000.0 / t2, 1),
                            "pairs": pair_count(scene),
                            "loss": "image.sum()" if grad is None else "dL/dimage N(0,1)"}
        out["extra"] = extra
        # the trainer's whole step on the 1080p bench scene
        out["train_step_bench_100k_1920x1080"] = train_steps(
            synthetic.bench_scene(n=N, width=1920, height=1080, device=dev), max(10, args.steps // 2))
    if not args.no_scale:
        # the HBM-bound stages where they move hundreds of MB: the per-Gaussian
        # kernels on config c5's 5M-Gaussian cloud, the depth sort and the
        # tile binning / LSD tile sort on config c4's 1M-Gaussian frame
        c5 = synthetic.config_scene("c5", device=dev, requires_grad=False)
        scale = {"per_gaussian_c5_5M": per_gaussian_stages(c5)}
        del c5
        c4 = synthetic.config_scene("c4", device=dev)
        scale["c4_1M_1920x1080"] = frame_stages(c4, 5)
        scale["adc_pass_c4_1M"] = adc_pass(c4)
        scale["c4_1M_1920x1080_tile_sort"] = frame_stages(c4, 5, binning="sort")
        del c4
        out["scale"] = scale
    if not args.no_c5:
        # config c5 (5M Gaussians, 3840x2160): ~1.1e10 pairs, beyond the int32
        # lists of the reference's surface, so rendered in screen bands
        c5 = synthetic.config_scene("c5", device=dev)
        out["c5_banded"] = banded_frame(c5, args.band_height or None, max(1, min(args.steps, 3)))
        del c5
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(sc)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
