"""bench.py's contract pieces that need no GPU: every stage the library times
has an algorithmic byte count, and --gpus above 1 is refused."""

from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def _timed_stages() -> set[str]:
    src = (ROOT / "custom-3dgs-cuda_amd" / "csrc" / "gsr_capi.cpp").read_text()
    return set(re.findall(r'StageTimer timer\("([a-z_]+)"', src))


def test_every_timed_stage_has_a_byte_count():
    stages = _timed_stages()
    assert {"blend_fwd", "blend_bwd", "project_sh", "project_sh_bwd"} <= stages
    for st in sorted(stages):
        b = bench.stage_bytes(st, 100_000, 13_000_000, 1920, 1080)
        assert b is not None and b > 0, st


def test_unknown_stage_has_no_byte_count():
    assert bench.stage_bytes("no_such_stage", 1, 1, 16, 16) is None


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(n)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "1 GPU" in (r.stdout + r.stderr)


@pytest.mark.parametrize("n, m, w, h, passes", [
    (10_000, 30_900, 256, 256, 5),          # c1: T = 256, ceil((32 + 8) / 8)
    (100_000, 1_810_000, 1280, 720, 6),     # c2: T = 3600, ceil((32 + 12) / 8)
    (100_000, 3_490_000, 1920, 1080, 6),    # c3: T = 8160, ceil((32 + 13) / 8)
    (1_000_000, 41_600_000, 3840, 2160, 6), # T = 32400, ceil((32 + 15) / 8)
])
def test_reference_binning_bytes_follow_the_fixed_formula(n, m, w, h, passes):
    t = ((w + 15) // 16) * ((h + 15) // 16)
    want = 64 * n + 12 * m + passes * 24 * m + 8 * m + 8 * t
    assert bench.reference_binning_bytes(n, m, w, h) == want


def test_binning_summary_sums_the_binning_stages_only():
    st = {"bin_count": {"ms": 0.02}, "depth_sort": {"ms": 0.03},
          "tile_binning": {"ms": 0.05}, "blend_fwd": {"ms": 0.2}}
    s = bench.binning_summary(st, 100_000, 13_000_000, 1920, 1080)
    assert s["stages"] == ["bin_count", "depth_sort", "tile_binning"]
    assert s["ms"] == pytest.approx(0.1)
    ref = bench.reference_binning_bytes(100_000, 13_000_000, 1920, 1080)
    assert s["reference_equiv_GBps"] == pytest.approx(ref / 1e-4 / 1e9, rel=1e-3)
