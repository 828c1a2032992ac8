"""ctypes front end of the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module; it is the checker, never the measured or shipped path.
Each wrapper names the reference file:line it restates (kmurungi/custom-3dgs-cuda).
Arrays are numpy, C-contiguous; ``dtype`` picks the fp32 (bit-exact reference
semantics) or fp64 (smooth math for finite-difference pins) instantiation.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
# GSR_ORACLE_LIB selects another build of the same source (the sanitizer
# build of tests/test_sanitizers.py)
_LIB_PATH = Path(os.environ.get("GSR_ORACLE_LIB", str(_HERE / "libgs_oracle.so")))
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")


def build(force: bool = False) -> Path:
    """Compile libgs_oracle.so with the Makefile beside this file."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-B" if force else "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        build()
    L = ctypes.CDLL(str(_LIB_PATH))
    c_int, c_f, c_d, c_i64 = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_int64
    vp = ctypes.c_void_p
    L.orc_expf.argtypes = [c_f]
    L.orc_expf.restype = c_f
    L.orc_expf_array.argtypes = [c_i64, _f32p, _f32p]
    L.orc_num_threads.restype = c_int
    L.orc_set_num_threads.argtypes = [c_int]
    L.orc_project_f32.argtypes = [c_int] + [_f32p] * 5 + [c_f] * 4 + [_f32p] * 3
    L.orc_project_f64.argtypes = [c_int] + [_f64p] * 5 + [c_d] * 4 + [_f64p] * 3
    L.orc_sh_f32.argtypes = [c_int] + [_f32p] * 5
    L.orc_sh_f64.argtypes = [c_int] + [_f64p] * 5
    L.orc_bin_count.argtypes = [c_int, _f32p, _f32p, c_int, c_int, _i32p, vp]
    L.orc_emit_keys.argtypes = [c_int, _f32p, _f32p, _f32p, c_int, c_int, vp, vp]
    L.orc_emit_keys.restype = c_i64
    L.orc_sort_pairs.argtypes = [c_i64, _u64p, _i32p]
    L.orc_tile_ranges.argtypes = [c_i64, _u64p, c_int, _i32p]
    L.orc_blend_fwd_f32.argtypes = [c_int, c_int, c_int, _i32p, _i32p] + [_f32p] * 6 + [_i32p]
    L.orc_blend_fwd_f64.argtypes = [c_int, c_int, c_int, _i32p, _i32p] + [_f64p] * 6 + [_i32p]
    L.orc_blend_bwd_f32.argtypes = [c_int, c_int, c_int] + [_f32p] * 5 + [_i32p, _i32p, _f32p, _i32p, _f64p, vp]
    L.orc_blend_bwd_f64.argtypes = [c_int, c_int, c_int] + [_f64p] * 5 + [_i32p, _i32p, _f64p, _i32p, _f64p, vp]
    L.orc_sh_bwd_f32.argtypes = [c_int] + [_f32p] * 8
    L.orc_sh_bwd_f64.argtypes = [c_int] + [_f64p] * 8
    L.orc_project_bwd_f32.argtypes = [c_int] + [_f32p] * 7 + [c_f] * 4 + [_f32p] * 3 + [c_int]
    L.orc_project_bwd_f64.argtypes = [c_int] + [_f64p] * 7 + [c_d] * 4 + [_f64p] * 3 + [c_int]
    L.orc_adam_step_f32.argtypes = [c_i64] + [_f32p] * 4 + [c_d] * 4 + [c_i64, c_f, c_f, c_int]
    _lib = L
    return L


def set_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().orc_num_threads())


def _c(a, dtype):
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def _sfx(dtype) -> str:
    return "f32" if np.dtype(dtype) == np.float32 else "f64"


def expf(x: float) -> float:
    """The build's fp32 exp (Cody–Waite + degree-6 polynomial), shared with the kernels."""
    return float(lib().orc_expf(float(x)))


def expf_array(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).ravel())
    y = np.empty_like(x)
    lib().orc_expf_array(x.size, x, y)
    return y


def project(mu, q, s, R, t, fx, fy, cx, cy, dtype=np.float32):
    """csrc/forward/projection.cu:12-107 -> (mean2d [N,2], cov2d [N,3], depth [N])."""
    mu, q, s, R, t = (_c(a, dtype) for a in (mu, q, s, R, t))
    n = mu.shape[0]
    mean2d = np.zeros((n, 2), dtype)
    cov2d = np.zeros((n, 3), dtype)
    depth = np.zeros((n,), dtype)
    getattr(lib(), "orc_project_" + _sfx(dtype))(n, mu, q, s, R, t, fx, fy, cx, cy, mean2d, cov2d, depth)
    return mean2d, cov2d, depth


def sh(cam, mu, A, kj, dtype=np.float32):
    """csrc/forward/SH.cu:57-93 -> colours [N,3] clamped to [0,1]."""
    cam, mu, A, kj = (_c(a, dtype) for a in (cam, mu, A, kj))
    n = mu.shape[0]
    out = np.zeros((n, 3), dtype)
    getattr(lib(), "orc_sh_" + _sfx(dtype))(n, cam, mu, A, kj, out)
    return out


def bin_count(mean2d, cov2d, H, W):
    """csrc/forward/rasterize.cu:7-61 -> (counts [N] i32, rect [N,4] = x0,x1,y0,y1 tiles)."""
    mean2d, cov2d = _c(mean2d, np.float32), _c(cov2d, np.float32)
    n = mean2d.shape[0]
    counts = np.zeros((n,), np.int32)
    rect = np.zeros((n, 4), np.int32)
    lib().orc_bin_count(n, mean2d, cov2d, int(H), int(W), counts, rect.ctypes.data_as(ctypes.c_void_p))
    return counts, rect


def emit_keys(mean2d, cov2d, depth, H, W):
    """csrc/forward/rasterize.cu:63-136 (+ the scan at :367-390) -> (keys u64 [M], ids i32 [M])."""
    mean2d, cov2d, depth = (_c(a, np.float32) for a in (mean2d, cov2d, depth))
    n = mean2d.shape[0]
    m = lib().orc_emit_keys(n, mean2d, cov2d, depth, int(H), int(W), None, None)
    keys = np.zeros((m,), np.uint64)
    ids = np.zeros((m,), np.int32)
    if m:
        lib().orc_emit_keys(n, mean2d, cov2d, depth, int(H), int(W),
                            keys.ctypes.data_as(ctypes.c_void_p), ids.ctypes.data_as(ctypes.c_void_p))
    return keys, ids


def sort_pairs(keys, ids):
    """Stable ascending sort on all 64 key bits (rasterize.cu:416-435)."""
    keys = np.array(keys, dtype=np.uint64, copy=True)
    ids = np.array(ids, dtype=np.int32, copy=True)
    if keys.size:
        lib().orc_sort_pairs(keys.size, keys, ids)
    return keys, ids


def tile_ranges(sorted_keys, T):
    """csrc/forward/rasterize.cu:140-166 -> ranges [T,2] i32, empty tiles (0,0)."""
    sk = _c(sorted_keys, np.uint64)
    out = np.zeros((T, 2), np.int32)
    lib().orc_tile_ranges(sk.size, sk, int(T), out)
    return out


def blend_fwd(ranges, ids, mean2d, cov2d, colors, alpha, H, W, dtype=np.float32):
    """csrc/forward/rasterize.cu:168-281 -> (img [H,W,3], final_T [H,W], n_contrib [H,W])."""
    ranges, ids = _c(ranges, np.int32), _c(ids, np.int32)
    mean2d, cov2d, colors, alpha = (_c(a, dtype) for a in (mean2d, cov2d, colors, alpha))
    n = mean2d.shape[0]
    img = np.zeros((H, W, 3), dtype)
    fT = np.ones((H, W), dtype)
    nc = np.zeros((H, W), np.int32)
    getattr(lib(), "orc_blend_fwd_" + _sfx(dtype))(n, H, W, ranges, ids, mean2d, cov2d, colors,
                                                    alpha.ravel(), img, fT, nc)
    return img, fT, nc


def rasterize(depth, mean2d, cov2d, colors, alpha, H, W):
    """The whole ``rasterize`` boundary (rasterize.cu:284-487), fp32.

    Returns (img, sorted_ids, tile_ranges, final_T, n_contrib, sorted_keys).
    """
    T = ((W + 15) // 16) * ((H + 15) // 16)
    n = np.asarray(mean2d).shape[0]
    keys, ids = emit_keys(mean2d, cov2d, depth, H, W) if n else (np.zeros(0, np.uint64), np.zeros(0, np.int32))
    if keys.size == 0:
        return (np.zeros((H, W, 3), np.float32), np.zeros(0, np.int32), np.zeros((T, 2), np.int32),
                np.ones((H, W), np.float32), np.zeros((H, W), np.int32), keys)
    skeys, sids = sort_pairs(keys, ids)
    ranges = tile_ranges(skeys, T)
    img, fT, nc = blend_fwd(ranges, sids, mean2d, cov2d, colors, alpha, H, W)
    return img, sids, ranges, fT, nc, skeys


def blend_bwd(grad, mean2d, cov2d, colors, alpha, ids, ranges, final_T, n_contrib, H, W,
              dtype=np.float32, with_abs=False):
    """csrc/backward/rasterize_backward.cu:6-236 with float64 accumulation.

    Returns (d_mean2d [N,2], d_cov2d [N,3], d_colors [N,3], d_alpha [N,1]) as float64,
    plus the matching sums of |term| when ``with_abs``.
    """
    grad, mean2d, cov2d, colors, alpha, final_T = (
        _c(a, dtype) for a in (grad, mean2d, cov2d, colors, alpha, final_T))
    ids, ranges, n_contrib = _c(ids, np.int32), _c(ranges, np.int32), _c(n_contrib, np.int32)
    n = mean2d.shape[0]
    acc = np.zeros((n, 9), np.float64)
    ab = np.zeros((n, 9), np.float64) if with_abs else None
    getattr(lib(), "orc_blend_bwd_" + _sfx(dtype))(
        n, H, W, grad, mean2d, cov2d, colors, alpha.ravel(), ids, ranges, final_T, n_contrib, acc,
        ab.ctypes.data_as(ctypes.c_void_p) if ab is not None else None)
    split = lambda a: (a[:, 0:2], a[:, 2:5], a[:, 5:8], a[:, 8:9])
    return split(acc) + (split(ab) if ab is not None else ())


def sh_bwd(cgrad, mu, A, kj, cam, dtype=np.float32):
    """csrc/backward/delight_backward.cu:107-174 -> (dA [N,3], dk_j [N,15,3], dmu [N,3])."""
    cgrad, mu, A, kj, cam = (_c(a, dtype) for a in (cgrad, mu, A, kj, cam))
    n = mu.shape[0]
    dA = np.zeros((n, 3), dtype)
    dkj = np.zeros((n, 15, 3), dtype)
    dmu = np.zeros((n, 3), dtype)
    getattr(lib(), "orc_sh_bwd_" + _sfx(dtype))(n, cgrad, mu, A, kj, cam, dA, dkj, dmu)
    return dA, dkj, dmu


def project_bwd(dmean, dcov, mu, q, s, R, t, fx, fy, cx, cy, dtype=np.float32, ref_quat=False):
    """csrc/backward/projection_backward.cu:11-140 -> (dmu [N,3], dq [N,4], ds [N,3]).

    ``ref_quat=True`` evaluates the reference's quaternion formula literally
    (projection_backward.cu:116-127), which fails finite differences; the default
    is the derivative of glm::toMat3 that the reference's own test demands.
    """
    dmean, dcov, mu, q, s, R, t = (_c(a, dtype) for a in (dmean, dcov, mu, q, s, R, t))
    n = mu.shape[0]
    dmu = np.zeros((n, 3), dtype)
    dq = np.zeros((n, 4), dtype)
    ds = np.zeros((n, 3), dtype)
    getattr(lib(), "orc_project_bwd_" + _sfx(dtype))(n, dmean, dcov, mu, q, s, R, t, fx, fy, cx, cy,
                                                      dmu, dq, ds, int(bool(ref_quat)))
    return dmu, dq, ds


def tiles(H: int, W: int) -> int:
    return ((W + 15) // 16) * ((H + 15) // 16)


def adam_step(p, g, m, v, lr, step, beta1=0.9, beta2=0.999, eps=1e-15, clamp_min=None,
              clamp_max=None, path="device"):
    """One Adam step with the trainer's clamps (utils/optim.py:12-31;
    scripts/train.py:171-176, utils/adc.py:90-93) on fp32 copies: returns
    (p, m, v) after the step (``step`` is the step number after the update, 1
    for the first).  ``path`` "device": torch.optim.Adam's default path on the
    GPU (multi-tensor); "cpu": its single-tensor path on the CPU."""
    if path not in ("device", "cpu"):
        raise ValueError("path must be 'device' or 'cpu'")
    p, m, v = (np.array(a, dtype=np.float32, copy=True, order="C").ravel() for a in (p, m, v))
    g = _c(g, np.float32).ravel()
    lo = np.float32(-np.inf if clamp_min is None else clamp_min)
    hi = np.float32(np.inf if clamp_max is None else clamp_max)
    lib().orc_adam_step_f32(p.size, p, g, m, v, float(lr), float(beta1), float(beta2), float(eps),
                            int(step), lo, hi, 1 if path == "device" else 0)
    return p, m, v
