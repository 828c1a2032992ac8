"""GPU tests of the boundary's modes and error paths:

- GSR_REFERENCE_QUAT_GRAD=1: backwards_projection and the fused tail give the
  reference's literal quaternion gradient (projection_backward.cu:116-127, the
  oracle's ref_quat mode) bit for bit, and d_mu / d_s do not change; read on
  every call, and also set before import in a fresh process;
- the device status word: an error bit raised on the device (the test hook,
  as a kernel at its spin bound would) makes the next rasterize raise, once;
- a list that holds one Gaussian twice in a tile (a caller-supplied list):
  the second entry has no gradient slot of its own and still counts, as in
  the reference's per-pixel atomics."""

from __future__ import annotations

import ctypes
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from gaussian_splatting import synthetic
from helpers import assert_bitwise, assert_grad_close, oracle_forward, scene_arrays
from oracle import oracle as orc
from test_gpu_parity import _dev, _np, gpu_forward

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "custom-3dgs-cuda_amd" / "libgsraster.so"


def _quat_case(n=50_000, seed=9):
    rng = np.random.default_rng(seed)
    a = scene_arrays(synthetic.config_scene("c3", requires_grad=False, n=n))
    a["mu"][::7, 2] = -1.0  # some culled Gaussians
    dm = rng.normal(size=(n, 2)).astype(np.float32)
    dc = rng.normal(size=(n, 3)).astype(np.float32)
    cg = rng.normal(size=(n, 3)).astype(np.float32)
    return a, dm, dc, cg


def test_reference_quaternion_gradient_mode(crc, device, monkeypatch):
    a, dm, dc, cg = _quat_case()
    d = {k: _dev(a[k], device) for k in ("mu", "q", "s", "R", "t", "A", "kj", "cam")}
    args = (_dev(dm, device), _dev(dc, device), d["mu"], d["q"], d["s"], d["R"], d["t"], a["fx"],
            a["fy"], a["cx"], a["cy"])
    true_mode = [_np(x) for x in crc.backwards_projection(*args)]
    monkeypatch.setenv("GSR_REFERENCE_QUAT_GRAD", "1")
    ref_mode = [_np(x) for x in crc.backwards_projection(*args)]
    fused = [_np(x) for x in crc.backwards_project_sh(
        _dev(dm, device), _dev(dc, device), _dev(cg, device), d["mu"], d["q"], d["s"], d["R"],
        d["t"], a["fx"], a["fy"], d["A"], d["kj"], d["cam"])]
    monkeypatch.delenv("GSR_REFERENCE_QUAT_GRAD")
    want_ref = orc.project_bwd(dm, dc, a["mu"], a["q"], a["s"], a["R"], a["t"], a["fx"], a["fy"],
                               a["cx"], a["cy"], ref_quat=True)
    want_true = orc.project_bwd(dm, dc, a["mu"], a["q"], a["s"], a["R"], a["t"], a["fx"],
                                a["fy"], a["cx"], a["cy"])
    assert_bitwise(ref_mode[1], want_ref[1], "d_q, reference mode")
    assert_bitwise(fused[1], want_ref[1], "fused tail d_q, reference mode")
    assert_bitwise(true_mode[1], want_true[1], "d_q, default mode")
    # the two modes differ in d_q only
    assert not np.array_equal(ref_mode[1], true_mode[1])
    assert_bitwise(ref_mode[0], true_mode[0], "d_mu unaffected")
    assert_bitwise(ref_mode[2], true_mode[2], "d_s unaffected")
    assert_bitwise(fused[2], true_mode[2], "fused tail d_s unaffected")
    w_sh = orc.sh_bwd(cg, a["mu"], a["A"], a["kj"], a["cam"])
    assert_bitwise(fused[0], (want_true[0] + w_sh[2]).astype(np.float32), "fused tail d_mu")


_FRESH = r"""
import sys
sys.path[:0] = [{root!r}, {pkg!r}, {tests!r}]
import numpy as np, torch
import custom_rasterizer_cuda as crc
from test_gpu_boundary import _quat_case
from oracle import oracle as orc
a, dm, dc, cg = _quat_case(n=20_000, seed=4)
dev = torch.device("cuda")
t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
got = crc.backwards_projection(t(dm), t(dc), t(a["mu"]), t(a["q"]), t(a["s"]), t(a["R"]),
                               t(a["t"]), a["fx"], a["fy"], a["cx"], a["cy"])
want = orc.project_bwd(dm, dc, a["mu"], a["q"], a["s"], a["R"], a["t"], a["fx"], a["fy"],
                       a["cx"], a["cy"], ref_quat=True)
for g, w in zip(got, want):
    assert np.array_equal(g.cpu().numpy().view(np.uint32), w.view(np.uint32)), "differs"
print("fresh-process reference quaternion gradient: bit-exact", flush=True)
"""


def test_reference_quaternion_gradient_mode_set_before_import(device):
    """The variable set in the environment of a new process before anything is
    imported, as a user of the reference's scripts would set it."""
    env = dict(os.environ, GSR_REFERENCE_QUAT_GRAD="1")
    code = _FRESH.format(root=str(ROOT), pkg=str(ROOT / "custom-3dgs-cuda_amd"),
                         tests=str(ROOT / "tests"))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "bit-exact" in r.stdout


def test_device_status_is_reported_once(crc, device):
    lib = ctypes.CDLL(str(LIB))
    lib.gsr_last_error.restype = ctypes.c_char_p
    sc = synthetic.config_scene("c1", requires_grad=False, n=2000, width=64, height=48)
    a = scene_arrays(sc)
    base = gpu_forward(crc, a, device)  # also leaves the status clear
    t = base["tensors"]
    n = a["mu"].shape[0]
    depth = _dev(oracle_forward(a)["depth"], device)
    args = (n, depth, t["mean2d"], t["cov2d"], t["colors"], t["alpha"], a["H"], a["W"])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # a bit raised on the device is reported by the next forward, and only once
    assert lib.gsr_debug_raise_status(1, stream) == 0, lib.gsr_last_error()
    with pytest.raises(RuntimeError, match="spin bound"):
        crc.rasterize(*args)
    again = crc.rasterize(*args)
    assert torch.equal(again[1], t["ids"])
    # ... and by the status call, which synchronizes
    assert lib.gsr_debug_raise_status(2, stream) == 0
    lib.gsr_rasterize_status.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    assert lib.gsr_rasterize_status(None, 0, stream) == 5
    assert b"inconsistent" in lib.gsr_last_error()
    assert lib.gsr_rasterize_status(None, 0, stream) == 0
    # a clean frame leaves nothing behind
    crc.rasterize(*args)
    assert lib.gsr_rasterize_status(None, 0, stream) == 0, lib.gsr_last_error()


def test_rasterize_backward_repeated_id_in_a_tile(crc, device):
    """Replace list entries with a copy of the entry before them (the same
    Gaussian twice in one tile, adjacent): the copies have no gradient slot of
    their own and take the atomic path; every contribution still counts."""
    a = scene_arrays(synthetic.config_scene("c1", requires_grad=False, n=3000, width=96,
                                            height=64))
    fw = gpu_forward(crc, a, device)
    want = oracle_forward(a)
    ids = want["ids"].copy()
    rng = want["ranges"]
    rg = np.random.default_rng(2)
    done = 0
    for t_ in range(rng.shape[0]):  # one copied entry in every tile with 3 or more
        s, e = rng[t_]
        if e - s >= 3:
            j = int(rg.integers(s + 1, e))
            ids[j] = ids[j - 1]
            done += 1
    assert done >= 20
    H, W, n = a["H"], a["W"], a["mu"].shape[0]
    G = synthetic.grad_image(H, W, seed=8).numpy()
    t = fw["tensors"]
    got = crc.backwards_rasterization(_dev(G, device), t["mean2d"], t["cov2d"], t["colors"],
                                      t["alpha"], _dev(ids, device, torch.int32), t["ranges"],
                                      t["final_T"], t["n_contrib"], n, H, W)
    torch.cuda.synchronize()
    ref = orc.blend_bwd(G, want["mean2d"], want["cov2d"], want["colors"], a["alpha"], ids,
                        want["ranges"], want["final_T"], want["n_contrib"], H, W, with_abs=True)
    for g, r, ab, nm in zip(got, ref[:4], ref[4:], ("d_mean2d", "d_cov2d", "d_colors", "d_alpha")):
        assert_grad_close(_np(g), r, ab, nm)
