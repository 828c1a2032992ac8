"""The C ABI (include/gsraster.h): every declared symbol is exported by libgsraster.so,
host-side validation works without a device, and (GPU) a ctypes call through the ABI
gives the same results as the pybind surface."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gsraster.h"
LIB = ROOT / "custom-3dgs-cuda_amd" / "libgsraster.so"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gsr_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    assert LIB.exists(), "libgsraster.so is not built (python custom-3dgs-cuda_amd/build.py)"
    L = ctypes.CDLL(str(LIB))
    L.gsr_last_error.restype = ctypes.c_char_p
    L.gsr_version.restype = ctypes.c_char_p
    L.gsr_build_sources.restype = ctypes.c_char_p
    L.gsr_bin_workspace_bytes.restype = ctypes.c_size_t
    L.gsr_bin_workspace_bytes.argtypes = [ctypes.c_int] * 3
    L.gsr_sort_workspace_bytes.restype = ctypes.c_size_t
    L.gsr_sort_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.gsr_backward_workspace_bytes.restype = ctypes.c_size_t
    L.gsr_backward_workspace_bytes.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int]
    return L


def test_header_declares_the_six_stages():
    names = _declared()
    for want in ("gsr_project", "gsr_sh", "gsr_rasterize_bin", "gsr_rasterize_render",
                 "gsr_rasterize_backward", "gsr_sh_backward", "gsr_project_backward"):
        assert want in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_library_names_the_sources_it_was_built_from(lib):
    """gsr_build_sources holds one sha256 prefix per source file; against the
    files in this tree it says whether the built library is current."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("gsr_build", ROOT / "custom-3dgs-cuda_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    text = lib.gsr_build_sources().decode()
    got = dict(item.split("=") for item in text.split(";"))
    assert {"gsr_blend.hip", "gsr_common.h", "gsr_capi.cpp", "gsraster.h"} <= set(got)
    assert all(len(h) == 16 and int(h, 16) >= 0 for h in got.values())
    assert got == mod.source_hashes(), "libgsraster.so is older than its sources: rebuild"


def test_host_side_queries_and_validation(lib):
    assert lib.gsr_version().decode().startswith("gsraster")
    assert lib.gsr_bin_workspace_bytes(100_000, 1080, 1920) > 100_000 * 48
    assert lib.gsr_sort_workspace_bytes(1_000_000, 100_000, 1080, 1920) >= 12_000_000
    assert lib.gsr_backward_workspace_bytes(10, 100, 32, 32) >= 480 + 2 * 4 * 4 + 36 * 100 + 100 // 8
    # n == 0 is a no-op; a null pointer with n > 0 is rejected before any HIP call
    assert lib.gsr_project(0, *([None] * 5), *([ctypes.c_float(1.0)] * 4), *([None] * 4)) == 0
    rc = lib.gsr_project(1, *([None] * 5), *([ctypes.c_float(1.0)] * 4), *([None] * 4))
    assert rc == 1 and b"null" in lib.gsr_last_error()
    rc = lib.gsr_rasterize_bin(-1, None, None, None, 16, 16, None, ctypes.c_size_t(0),
                               ctypes.byref(ctypes.c_int64()), None)
    assert rc == 1


def test_extension_module_surface():
    import sys
    sys.path.insert(0, str(ROOT / "custom-3dgs-cuda_amd"))
    import torch
    import custom_rasterizer_cuda as crc

    for name in ("project", "SH", "rasterize", "backwards_rasterization", "backwards_SH",
                 "backwards_projection"):
        assert callable(getattr(crc, name))
    with pytest.raises(RuntimeError, match="mu3d must be a CUDA tensor"):
        crc.project(1, torch.zeros(1, 3), torch.zeros(1, 4), torch.zeros(1, 3), torch.eye(3),
                    torch.zeros(3), 1.0, 1.0, 0.0, 0.0)


def test_rasterize_glue_reports_cpu_tensors():
    from gaussian_splatting import synthetic
    from gaussian_splatting.rasterizer.rasterize import rasterize

    sc = synthetic.bench_scene(n=10, width=32, height=32)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        rasterize(sc.gaussians, sc.view)


@pytest.mark.gpu
def test_c_abi_project_matches_extension(lib, crc, device):
    import torch

    rng = np.random.default_rng(0)
    n = 4096
    mu = torch.from_numpy(np.c_[rng.uniform(-1, 1, (n, 2)), rng.uniform(1, 5, n)].astype(np.float32)).to(device)
    q = torch.from_numpy(rng.normal(size=(n, 4)).astype(np.float32)).to(device)
    s = torch.from_numpy(rng.normal(-3, 0.5, (n, 3)).astype(np.float32)).to(device)
    R, T = torch.eye(3, device=device), torch.zeros(3, device=device)
    want = crc.project(n, mu, q, s, R, T, 300.0, 300.0, 160.0, 120.0)
    out = [torch.empty(n, 2, device=device), torch.empty(n, 3, device=device), torch.empty(n, device=device)]
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    f = [ctypes.c_float(v) for v in (300.0, 300.0, 160.0, 120.0)]
    rc = lib.gsr_project(n, vp(mu), vp(q), vp(s), vp(R), vp(T), *f, *(vp(o) for o in out), stream)
    assert rc == 0, lib.gsr_last_error()
    torch.cuda.synchronize()
    for a, b in zip(out, want):
        assert torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("binning", ["blocks", "sort"])
def test_c_abi_rasterize_matches_extension_and_reports_no_error(lib, crc, device, monkeypatch,
                                                                 binning):
    """gsr_rasterize_bin + gsr_rasterize_render through ctypes give the extension's
    sorted ids, tile ranges and image, and gsr_rasterize_status then finds no
    device-side error (look-back spin bound, inconsistent counts)."""
    import torch

    from gaussian_splatting import synthetic

    if binning == "sort":
        monkeypatch.setenv("GSR_TILE_BINNING", "sort")
    sc = synthetic.config_scene("c3", requires_grad=False, n=20_000, width=480, height=270,
                                device=device)
    g, v = sc.gaussians, sc.view
    n, H, W = g.mu.shape[0], int(v["height"]), int(v["width"])
    mean2d, cov2d, depth = crc.project(n, g.mu.contiguous(), g.q.contiguous(), g.s.contiguous(),
                                       v["R"].contiguous(), v["T"].contiguous(), float(v["fx"]),
                                       float(v["fy"]), float(v["cx"]), float(v["cy"]))
    cam = crc.camera_position(v["R"].contiguous(), v["T"].contiguous())
    colors = crc.SH(n, cam, g.mu.contiguous(), g.A.contiguous(), g.k_j.contiguous())
    alpha = torch.sigmoid(g.alpha).contiguous().reshape(-1)
    img_w, ids_w, rng_w, _, _, _ = crc.rasterize_with_keys(n, depth, mean2d, cov2d, colors,
                                                           alpha, H, W)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sz, i64 = ctypes.c_size_t, ctypes.c_int64
    T = ((W + 15) // 16) * ((H + 15) // 16)
    bb = lib.gsr_bin_workspace_bytes(n, H, W)
    bws = torch.empty(bb, dtype=torch.uint8, device=device)
    m = i64()
    lib.gsr_rasterize_bin.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [
        ctypes.c_int, ctypes.c_int, ctypes.c_void_p, sz, ctypes.POINTER(i64), ctypes.c_void_p]
    rc = lib.gsr_rasterize_bin(n, vp(depth), vp(mean2d), vp(cov2d), H, W, vp(bws), bb,
                               ctypes.byref(m), stream)
    assert rc == 0, lib.gsr_last_error()
    assert m.value == ids_w.numel()
    sb = lib.gsr_sort_workspace_bytes(m.value, n, H, W)
    sws = torch.empty(sb, dtype=torch.uint8, device=device)
    ids = torch.empty(m.value, dtype=torch.int32, device=device)
    ranges = torch.full((T, 2), -7, dtype=torch.int32, device=device)
    img = torch.empty(H, W, 3, device=device)
    fT = torch.empty(H, W, device=device)
    nc = torch.empty(H, W, dtype=torch.int32, device=device)
    lib.gsr_rasterize_render.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 5 + [
        ctypes.c_int, ctypes.c_int, ctypes.c_void_p, sz, i64, ctypes.c_void_p, sz] + \
        [ctypes.c_void_p] * 7
    rc = lib.gsr_rasterize_render(n, vp(depth), vp(mean2d), vp(cov2d), vp(colors), vp(alpha),
                                  H, W, vp(bws), bb, m.value, vp(sws), sb, vp(ids), vp(ranges),
                                  vp(img), vp(fT), vp(nc), None, stream)
    assert rc == 0, lib.gsr_last_error()
    lib.gsr_rasterize_status.argtypes = [ctypes.c_void_p, sz, ctypes.c_void_p]
    assert lib.gsr_rasterize_status(vp(bws), bb, stream) == 0, lib.gsr_last_error()
    torch.cuda.synchronize()
    assert torch.equal(ids, ids_w)
    assert torch.equal(ranges, rng_w.reshape(T, 2))
    assert torch.equal(img, img_w.reshape(H, W, 3))
