"""Build libgsraster.so (HIP, gfx950) and the custom_rasterizer_cuda module in place.

    python custom-3dgs-cuda_amd/build.py [--jobs N]

libgsraster.so: every csrc/*.hip plus csrc/gsr_capi.cpp, compiled by hipcc with
--offload-arch=gfx950, -ffp-contract=off (the fp32 forward keeps the reference's
operation order; see csrc/gsr_common.h), packed-fp32 instructions disabled, and
-munsafe-fp-atomics: the backward's few float atomics (list entries without a
gradient slot of their own) use the hardware's float add.
custom_rasterizer_cuda*.so: csrc/bindings.cpp compiled against torch's headers and
linked to libgsraster.so (rpath $ORIGIN).
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
INCLUDE = PKG.parent / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = os.environ.get("GSR_OFFLOAD_ARCH", "gfx950")

LIB = PKG / "libgsraster.so"
EXT = PKG / ("custom_rasterizer_cuda" + sysconfig.get_config_var("EXT_SUFFIX"))

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        # hipcc's host pass does not know the device-only feature flag
        if "packed-fp32-ops" not in line and "unknown target feature" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip() and os.environ.get("GSR_BUILD_VERBOSE"):
        print(out)


def code_of(text: str) -> str:
    """C/C++ source without its comments, blank lines and runs of blanks: what
    an edit has to change to change the compiled code.  String and character
    literals are kept as they are."""
    out, i, n = [], 0, len(text)
    while i < n:
        c = text[i]
        if c in "\"'":
            j = i + 1
            while j < n and text[j] != c:
                j += 2 if text[j] == "\\" else 1
            out.append(text[i:j + 1])
            i = j + 1
        elif text.startswith("//", i):
            while i < n and text[i] != "\n":
                i += 1
        elif text.startswith("/*", i):
            j = text.find("*/", i + 2)
            i = n if j < 0 else j + 2
            out.append(" ")
        else:
            out.append(c)
            i += 1
    lines = (" ".join(line.split()) for line in "".join(out).splitlines())
    return "\n".join(line for line in lines if line)


def source_hashes() -> dict[str, str]:
    """The first 16 hex digits of the sha256 of the code (code_of) of every
    file the library is built from.  The library returns them
    (gsr_build_sources) so that a measurement can name the code it measured and
    a later run can tell whether it changed; edits to comments alone change no
    hash."""
    files = (sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + [CSRC / "gsr_capi.cpp"]
             + [INCLUDE / "gsraster.h"])
    return {f.name: hashlib.sha256(code_of(f.read_text()).encode()).hexdigest()[:16]
            for f in files}


def _sources_define() -> str:
    text = ";".join(f"{k}={v}" for k, v in source_hashes().items())
    return f'-DGSR_SOURCES="{text}"'


def _hip_objects(jobs: int) -> list[Path]:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + [CSRC / "gsr_capi.cpp"]
    objs = []
    cmds = []
    for src in sources:
        obj = BUILD / (src.name + ".o")
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        extra = [_sources_define()] if src.name == "gsr_capi.cpp" else []
        cmds.append([HIPCC, *HIP_FLAGS, *lang, *extra, "-c", str(src), "-o", str(obj)])
        objs.append(obj)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    return objs


def build_library(jobs: int = 8) -> Path:
    objs = _hip_objects(jobs)
    tmp = LIB.with_suffix(".so.tmp")
    # -z defs: an undefined symbol fails the link, not the first import
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *map(str, objs),
          "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


SAN_DIR = BUILD / "san"
SAN_LIB = SAN_DIR / "libgsraster_hostsan.so"


def build_host_sanitized() -> Path:
    """libgsraster with its host code (the C ABI: argument checks, layouts,
    launches) under AddressSanitizer and UndefinedBehaviorSanitizer, for the
    CPU tests in tests/test_sanitizers.py.  Only gsr_capi.cpp is recompiled
    (host code only, the sanitizers passed with -Xarch_host so no device code
    is instrumented); the kernels' objects are the ones build_library made."""
    objs = sorted(BUILD.glob("*.hip.o"))
    if not objs:
        raise RuntimeError("build the library first (its kernel objects are reused)")
    SAN_DIR.mkdir(parents=True, exist_ok=True)
    capi = SAN_DIR / "gsr_capi_san.o"
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g"]
    _run([HIPCC, *[f for f in HIP_FLAGS if f != "-O3"], "-O1", *san, _sources_define(), "-c",
          str(CSRC / "gsr_capi.cpp"), "-o", str(capi)])
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *san, *map(str, objs), str(capi),
          "-o", str(SAN_LIB)])
    return SAN_LIB


def build_extension() -> Path:
    import torch
    from torch.utils.cpp_extension import include_paths, library_paths

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{p}" for p in include_paths()] + [
        f"-I{sysconfig.get_paths()['include']}", f"-I{ROCM / 'include'}", f"-I{INCLUDE}"]
    libdirs = library_paths()
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=custom_rasterizer_cuda",
        "-Wno-deprecated-declarations",
        *inc, str(CSRC / "bindings.cpp"),
        *[f"-L{d}" for d in libdirs], f"-L{PKG}", f"-L{ROCM / 'lib'}",
        "-lgsraster", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-ltorch_python", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs],
        "-o", str(EXT.with_suffix(".tmp")),
    ]
    _run(cmd)
    os.replace(EXT.with_suffix(".tmp"), EXT)
    return EXT


def build(jobs: int = 8) -> tuple[Path, Path]:
    lib = build_library(jobs)
    ext = build_extension()
    return lib, ext


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--lib-only", action="store_true", help="build libgsraster.so only")
    ap.add_argument("--clean", action="store_true", help="remove _build/ first")
    args = ap.parse_args()
    if args.clean and BUILD.exists():
        shutil.rmtree(BUILD)
    lib = build_library(args.jobs)
    print(f"built {lib}")
    if not args.lib_only:
        print(f"built {build_extension()}")


if __name__ == "__main__":
    sys.exit(main())
