"""gsr_rasterize_backward_noalloc: the backward for callers that cannot allocate,
with its workspace in the library's fixed per-device scratch array.  Through
the C ABI it gives gsr_rasterize_backward's outputs bit for bit, on two calls
in a row (the second with a smaller frame, so that what the first left in
the shared array must not leak into it), and it rejects a frame whose
workspace exceeds the array."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from gaussian_splatting import synthetic
from helpers import assert_bitwise, scene_arrays
from test_gpu_parity import _dev, _np, gpu_forward

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "custom-3dgs-cuda_amd" / "libgsraster.so"
SCRATCH = 256 << 20  # GSR_NOALLOC_SCRATCH_BYTES


def _lib():
    L = ctypes.CDLL(str(LIB))
    L.gsr_last_error.restype = ctypes.c_char_p
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    L.gsr_backward_workspace_bytes.restype = sz
    L.gsr_backward_workspace_bytes.argtypes = [i32, i64, i32, i32]
    L.gsr_rasterize_backward.argtypes = [i32, i32, i32] + [vp] * 6 + [i64] + [vp] * 3 + \
        [vp, sz] + [vp] * 4 + [vp]
    L.gsr_rasterize_backward_noalloc.argtypes = [i32, i32, i32] + [vp] * 6 + [i64] + \
        [vp] * 3 + [vp] * 4 + [vp]
    return L


def _frame(crc, device, name, **kw):
    a = scene_arrays(synthetic.config_scene(name, requires_grad=False, **kw))
    fw = gpu_forward(crc, a, device)
    G = _dev(synthetic.grad_image(a["H"], a["W"], seed=6).numpy(), device)
    return a, fw["tensors"], G


def _run(L, a, t, G, device, noalloc):
    n, H, W = a["mu"].shape[0], a["H"], a["W"]
    m = t["ids"].numel()
    vp = lambda x: ctypes.c_void_p(x.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = [torch.full((n, 2), 7.0, device=device), torch.full((n, 3), 7.0, device=device),
           torch.full((n, 3), 7.0, device=device), torch.full((n,), 7.0, device=device)]
    common = (n, H, W, vp(G), vp(t["mean2d"]), vp(t["cov2d"]), vp(t["colors"]), vp(t["alpha"]),
              vp(t["ids"]), m, vp(t["ranges"]), vp(t["final_T"]), vp(t["n_contrib"]))
    if noalloc:
        rc = L.gsr_rasterize_backward_noalloc(*common, *(vp(o) for o in out), stream)
    else:
        wsb = L.gsr_backward_workspace_bytes(n, m, H, W)
        ws = torch.empty(wsb, dtype=torch.uint8, device=device)
        rc = L.gsr_rasterize_backward(*common, vp(ws), wsb, *(vp(o) for o in out), stream)
    assert rc == 0, L.gsr_last_error()
    torch.cuda.synchronize()
    return [_np(o) for o in out]


def test_noalloc_backward_matches_the_workspace_entry_point(crc, device):
    L = _lib()
    big = _frame(crc, device, "c3")  # 100k Gaussians at 1920x1080, ~3.5M pairs
    small = _frame(crc, device, "c1", n=3000, width=128, height=96)
    a, t, _ = big
    need = L.gsr_backward_workspace_bytes(a["mu"].shape[0], t["ids"].numel(), a["H"], a["W"])
    assert SCRATCH // 4 < need <= SCRATCH, need  # the first call fills much of the array
    for name, (a, t, G) in (("first, larger frame", big), ("second, smaller frame", small)):
        print(f"[gpu] no-alloc backward: {name}, {t['ids'].numel()} pairs", flush=True)
        got = _run(L, a, t, G, device, noalloc=True)
        want = _run(L, a, t, G, device, noalloc=False)
        for x, y, nm in zip(got, want, ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
            assert np.isfinite(x).all(), nm
            assert_bitwise(x, y, f"{name}: {nm}")


def test_noalloc_backward_rejects_frames_beyond_the_scratch(device):
    L = _lib()
    n, H, W = 100_000, 1080, 1920
    m = 20_000_000  # 36 B per pair: ~720 MB of workspace
    assert L.gsr_backward_workspace_bytes(n, m, H, W) > SCRATCH
    dummy = torch.zeros(16, device=device)
    p = ctypes.c_void_p(dummy.data_ptr())
    rc = L.gsr_rasterize_backward_noalloc(n, H, W, *([p] * 6), m, *([p] * 3), *([p] * 4), None)
    assert rc == 3  # GSR_ERR_WORKSPACE, before any launch
    assert b"scratch" in L.gsr_last_error()
