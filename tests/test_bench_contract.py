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


def test_valu_peak_is_the_published_fp32_figure_per_packed_wave64_fma():
    # 157.3 TFLOP/s fp32 / (64 lanes x 2 flops x 2 packed) = 614.4 G issues/s
    assert bench.VALU_PEAK_GISSUE == pytest.approx(157.3e12 / 256 / 1e9, rel=1e-3)


SOURCES = {f: "%016x" % i for i, f in enumerate(
    ("gsr_blend.hip", "gsr_tiles.hip", "gsr_bin.hip") + bench.SHARED_SOURCES)}


def _fake_profiles(monkeypatch, traffic=None, valu=None, library=None):
    """Profiles recorded on SOURCES; the loaded library built from ``library``
    (default: the same sources)."""
    for prof in (traffic, valu):
        if prof is not None:
            prof.setdefault("sources", dict(SOURCES))

    def fake(kind, workload):
        return {"traffic": traffic, "valu": valu}.get(kind)
    monkeypatch.setattr(bench, "_profile_json", fake)
    monkeypatch.setattr(bench, "library_sources", lambda: dict(library or SOURCES))


def test_stage_rates_use_measured_bytes_and_never_a_formula_for_the_blends(monkeypatch):
    _fake_profiles(monkeypatch, traffic={"stages": {"blend_bwd": {"bytes_per_call": 1.5e8},
                                                    "tile_binning": {"bytes_per_call": 1.1e8}}})
    st = {"blend_bwd": (10, 2.5), "blend_fwd": (10, 1.8), "tile_binning": (10, 0.5),
          "bin_count": (10, 0.2)}
    r = bench._stage_rates(st, 100_000, 13_000_000, 1920, 1080, workload="w")
    assert r["blend_bwd"]["bytes"] == "measured" and r["blend_bwd"]["bound"] == "valu"
    assert r["blend_bwd"]["GBps"] == pytest.approx(1.5e8 / 0.25e-3 / 1e9, rel=1e-3)
    # no measured traffic for the forward blend: no HBM rate at all
    assert r["blend_fwd"]["pct_hbm_peak"] is None and r["blend_fwd"]["bound"] == "valu"
    assert r["tile_binning"]["bytes"] == "measured"
    assert r["bin_count"]["bytes"] == "formula"
    assert r["bin_count"]["GBps"] == pytest.approx(
        bench.stage_bytes("bin_count", 100_000, 13_000_000, 1920, 1080) / 0.02e-3 / 1e9, rel=1e-3)


def test_blend_roofline_is_valu_issue_from_the_profile(monkeypatch):
    _fake_profiles(monkeypatch, traffic={"stages": {"blend_bwd": {"bytes_per_call": 1.46e8}}},
                   valu={"kernels": {"blend_bwd": {"issue_quads_per_launch": 1.255e8,
                                                   "insts_per_launch": 1.55e8,
                                                   "issue_util": 0.816, "clock_mhz": 2253}},
                         "calibration": {"fma": {"issue_util": 0.938}}})
    per = {"blend_bwd": {"ms": 0.257}}
    r = bench.dominant_roofline("blend_bwd", per, 100_000, 13_482_333, 1920, 1080, "w")
    assert r["bound"] == "valu" and r["peak"] == bench.VALU_PEAK_GISSUE
    assert r["achieved"] == pytest.approx(1.255e8 / 0.257e-3 / 1e9, rel=1e-3)
    assert r["frac"] == pytest.approx(r["achieved"] / bench.VALU_PEAK_GISSUE, rel=1e-3)
    assert r["traffic"] == 1.46e8 and r["hbm_measured"]["frac"] < 0.2
    assert r["equivalent"]["bytes"] == bench.stage_bytes("blend_bwd", 100_000, 13_482_333,
                                                          1920, 1080)
    assert r["calibration_issue_util"] == {"fma": 0.938}


def test_committed_profiles_cover_the_bench_roofline():
    t = bench._profile_json("traffic", "bench_100k_1920x1080")
    v = bench._profile_json("valu", "bench_100k_1920x1080")
    assert t and t["stages"]["blend_bwd"]["bytes_per_call"] > 0
    assert v and v["kernels"]["blend_bwd"]["issue_quads_per_launch"] > 0
    assert 0 < v["kernels"]["blend_bwd"]["issue_util"] <= 1.0
    for c in v["calibration"].values():
        assert 0.8 < c["issue_util"] <= 1.0


def _tree_sources():
    import importlib.util
    spec = importlib.util.spec_from_file_location("gsr_build", ROOT / "custom-3dgs-cuda_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.source_hashes()


PROFILE_JSONS = ("traffic_bench_100k_1920x1080", "traffic_c4_1000000_1920x1080_randn_grad",
                 "traffic_c4_1000000_1920x1080_randn_grad_tile_sort", "valu_bench_100k_1920x1080",
                 "valu_per_gaussian_c5_5M")


@pytest.mark.parametrize("name", PROFILE_JSONS)
def test_committed_profiles_were_measured_on_these_sources(monkeypatch, name):
    """Every stage or kernel entry of the committed profiles names its source
    files, and they (with the shared sources) hash as in this tree: the
    counters bench.py uses describe the kernels that are built here."""
    kind, workload = name.split("_", 1)
    prof = bench._profile_json(kind, workload)
    assert prof and set(prof["sources"]) == set(_tree_sources())
    monkeypatch.setattr(bench, "library_sources", _tree_sources)
    entries = prof["stages"] if kind == "traffic" else prof["kernels"]
    assert entries
    for key, entry in entries.items():
        assert entry["source_files"], key
        assert bench.stale_reason(prof, entry) is None, (key, bench.stale_reason(prof, entry))


def _changed(name):
    out = dict(SOURCES)
    out[name] = "f" * 16
    return out


def test_profiles_of_changed_sources_give_no_valu_fraction(monkeypatch):
    """A blend profile measured on other gsr_blend.hip code: frac is null with the
    reason, and the measured traffic is not used."""
    _fake_profiles(monkeypatch,
                   traffic={"stages": {"blend_bwd": {"bytes_per_call": 1.46e8,
                                                     "source_files": ["gsr_blend.hip"]}}},
                   valu={"kernels": {"blend_bwd": {"issue_quads_per_launch": 1.255e8,
                                                   "source_files": ["gsr_blend.hip"]}}},
                   library=_changed("gsr_blend.hip"))
    r = bench.dominant_roofline("blend_bwd", {"blend_bwd": {"ms": 0.25}}, 100_000,
                                13_000_000, 1920, 1080, "w")
    assert r["frac"] is None and r["achieved"] is None and r["traffic"] is None
    assert "gsr_blend.hip" in r["reason"]


def test_a_shared_header_change_also_makes_a_profile_stale(monkeypatch):
    _fake_profiles(monkeypatch,
                   valu={"kernels": {"blend_fwd": {"issue_quads_per_launch": 1e8,
                                                   "source_files": ["gsr_blend.hip"]}}},
                   library=_changed("gsr_common.h"))
    r = bench.dominant_roofline("blend_fwd", {"blend_fwd": {"ms": 0.2}}, 100_000,
                                13_000_000, 1920, 1080, "w")
    assert r["frac"] is None and "gsr_common.h" in r["reason"]


def test_a_profile_without_hashes_is_not_trusted(monkeypatch):
    _fake_profiles(monkeypatch, valu={"sources": {}, "kernels": {
        "blend_bwd": {"issue_quads_per_launch": 1e8}}})
    r = bench.dominant_roofline("blend_bwd", {"blend_bwd": {"ms": 0.2}}, 100_000,
                                13_000_000, 1920, 1080, "w")
    assert r["frac"] is None and "no source hashes" in r["reason"]


def test_stage_rates_fall_back_to_formula_bytes_for_changed_kernels(monkeypatch):
    """Only the stage whose kernel file changed loses its measured bytes."""
    _fake_profiles(monkeypatch, traffic={"stages": {
        "tile_binning": {"bytes_per_call": 1.1e8, "source_files": ["gsr_tiles.hip"]},
        "bin_count": {"bytes_per_call": 2.0e7, "source_files": ["gsr_bin.hip"]}}},
        library=_changed("gsr_tiles.hip"))
    st = {"tile_binning": (10, 0.5), "bin_count": (10, 0.2)}
    r = bench._stage_rates(st, 100_000, 13_000_000, 1920, 1080, workload="w")
    assert r["tile_binning"]["bytes"] == "formula"
    assert "gsr_tiles.hip" in r["tile_binning"]["measured_bytes_not_used"]
    assert r["bin_count"]["bytes"] == "measured"
    assert "measured_bytes_not_used" not in r["bin_count"]
