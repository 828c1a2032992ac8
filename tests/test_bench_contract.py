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
