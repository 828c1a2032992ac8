"""Pins of the shared fp32 exp (oracle/gs_oracle.cpp orc_expf; the kernels' exp_gs).

The reference calls CUDA's __expf / expf (rasterize.cu:255, rasterize_backward.cu:131,
projection.cu:70-72).  The build fixes one faithfully rounded exp on host and
device; these tests hold it to <= 1 ulp of the float64 exp and to IEEE special cases.
"""

import numpy as np


def _ulp_err(y32, x32):
    t = np.exp(x32.astype(np.float64))
    ulp = np.spacing(t.astype(np.float32)).astype(np.float64)
    return np.abs(y32.astype(np.float64) - t) / ulp


def test_exp_dense_sweep_is_faithful(orc):
    x = np.linspace(-87.3, 88.7, 2_000_003, dtype=np.float32)
    assert _ulp_err(orc.expf_array(x), x).max() < 1.0


def test_exp_near_zero_and_blend_range(orc):
    # the blend evaluates exp(power) with power in [-6, 0]; projection exp(log-scale)
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-6.0, 0.0, 500_000), rng.uniform(-1e-3, 1e-3, 100_000),
                        rng.normal(-3.0, 2.0, 200_000)]).astype(np.float32)
    assert _ulp_err(orc.expf_array(x), x).max() < 1.0


def test_exp_special_values(orc):
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-0.0) == 1.0
    assert orc.expf(89.0) == float("inf")
    assert orc.expf(float("inf")) == float("inf")
    assert orc.expf(-float("inf")) == 0.0
    assert orc.expf(-100.0) == 0.0
    assert np.isnan(orc.expf(float("nan")))
    # results below FLT_MIN flush to +0 and the cut sits at ln(FLT_MIN)
    assert orc.expf(-87.34) == 0.0
    assert orc.expf(-87.33) >= np.finfo(np.float32).tiny


def test_exp_monotone_on_blend_range(orc):
    # monotone exp keeps the alpha >= 1/255 decision consistent with power order
    x = np.sort(np.random.default_rng(1).uniform(-10.0, 0.0, 300_000).astype(np.float32))
    y = orc.expf_array(x)
    assert np.all(np.diff(y) >= 0)
