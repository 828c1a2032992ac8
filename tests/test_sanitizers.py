"""CPU-only sanitizer runs (AddressSanitizer + UndefinedBehaviorSanitizer).

- The oracle (oracle/gs_oracle.cpp) built with gcc's sanitizers
  (`make -C oracle san`) runs every oracle-side CPU test in a subprocess that
  preloads the ASan runtime; any UB report aborts (-fno-sanitize-recover).
- The C ABI's host code (gsr_capi.cpp: argument checks, workspace layouts)
  built with clang's sanitizers on the host side only (-Xarch_host; the kernels
  are the regular objects) answers size queries over edge-case shapes and
  rejects invalid calls, all before any HIP call, in a subprocess that
  preloads clang's ASan runtime.
Nothing here touches a GPU.
"""

from __future__ import annotations

import importlib.util
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "custom-3dgs-cuda_amd"
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _gcc_asan() -> str:
    out = subprocess.run(["g++", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    if out.returncode != 0 or not Path(path).is_file():
        pytest.skip("gcc's libasan is not installed")
    return path


def _clang_asan() -> str:
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    found = sorted(rocm.glob("llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        pytest.skip("clang's ASan runtime is not installed")
    return str(found[-1])


def _env(preload: str, **extra) -> dict:
    env = dict(os.environ)
    env.update(LD_PRELOAD=preload, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", **extra)
    return env


def _check(proc: subprocess.CompletedProcess, what: str) -> None:
    text = proc.stdout + proc.stderr
    bad = [ln for ln in text.splitlines() if any(r in ln for r in REPORTS)]
    assert not bad, f"{what}: sanitizer report\n" + "\n".join(bad[:20])
    assert proc.returncode == 0, f"{what}: exit {proc.returncode}\n{text[-3000:]}"


def test_oracle_under_asan_and_ubsan():
    asan = _gcc_asan()
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "san"], check=True)
    lib = ROOT / "oracle" / "_san" / "libgs_oracle.so"
    # the oracle's own tests and the CPU tests that run it (never this module)
    files = sorted(str(p) for p in (ROOT / "tests").glob("test_oracle_*.py"))
    files += [str(ROOT / "tests" / f) for f in ("test_ply.py", "test_bands.py")]
    proc = subprocess.run(
        [sys.executable, "-m", "pytest", *files, "-m", "not gpu", "-q", "-x",
         "-p", "no:cacheprovider"],
        cwd=ROOT, capture_output=True, text=True, timeout=900,
        env=_env(asan, GSR_ORACLE_LIB=str(lib)))
    _check(proc, "oracle tests under ASan/UBSan")
    assert " passed" in proc.stdout


_CAPI_SCRIPT = r"""
import ctypes, sys
L = ctypes.CDLL(sys.argv[1])
assert any('_build/san/' in l for l in open('/proc/self/maps')), 'sanitized library not mapped'
c_int, c_i64, c_sz, c_f = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
L.gsr_last_error.restype = ctypes.c_char_p
L.gsr_version.restype = ctypes.c_char_p
assert L.gsr_version().startswith(b'gsraster')
L.gsr_bin_workspace_bytes.restype = c_sz
L.gsr_bin_workspace_bytes.argtypes = [c_int] * 3
L.gsr_sort_workspace_bytes.restype = c_sz
L.gsr_sort_workspace_bytes.argtypes = [c_i64, c_int, c_int, c_int]
L.gsr_backward_workspace_bytes.restype = c_sz
L.gsr_backward_workspace_bytes.argtypes = [c_int, c_i64, c_int, c_int]
L.gsr_depth_order_workspace_bytes.restype = c_sz
L.gsr_depth_order_workspace_bytes.argtypes = [c_int]
shapes = [(0, 0, 0), (1, 1, 1), (100_000, 1080, 1920), (5_000_000, 2160, 3840),
          (3, 17, 33), (2**31 - 1, 16, 16), (-1, 16, 16), (10, -1, 5)]
for n, h, w in shapes:
    L.gsr_bin_workspace_bytes(n, h, w)
    L.gsr_depth_order_workspace_bytes(n)
    for m in (0, 1, 13_482_333, 2**31 - 65536, -1):
        L.gsr_sort_workspace_bytes(m, n, h, w)
        L.gsr_backward_workspace_bytes(n, m, h, w)
assert L.gsr_bin_workspace_bytes(10, -1, 5) == 0 and L.gsr_depth_order_workspace_bytes(-1) == 0
# invalid calls are rejected before any HIP call
assert L.gsr_project(0, *([None] * 5), *([c_f(1.0)] * 4), *([None] * 4)) == 0
assert L.gsr_project(1, *([None] * 5), *([c_f(1.0)] * 4), *([None] * 4)) == 1
assert b'null' in L.gsr_last_error()
assert L.gsr_rasterize_bin(-1, None, None, None, 16, 16, None, c_sz(0),
                           ctypes.byref(c_i64()), None) == 1
assert L.gsr_rasterize_bin(5, None, None, None, -16, 16, None, c_sz(0),
                           ctypes.byref(c_i64()), None) == 1
assert len(L.gsr_last_error()) > 0
print('capi host checks ok')
"""


def test_c_abi_host_code_under_asan_and_ubsan():
    asan = _clang_asan()
    if not sorted((PKG / "_build").glob("*.hip.o")):
        pytest.skip("the library's kernel objects are not built (custom-3dgs-cuda_amd/build.py)")
    spec = importlib.util.spec_from_file_location("gsr_build", PKG / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    lib = mod.build_host_sanitized()
    proc = subprocess.run([sys.executable, "-c", _CAPI_SCRIPT, str(lib)], cwd=ROOT,
                          capture_output=True, text=True, timeout=300, env=_env(asan))
    _check(proc, "C ABI host code under ASan/UBSan")
    assert "capi host checks ok" in proc.stdout
