"""Pins the repo-defined binary32 log and the saturating float->int conversion
shared by the oracle and the kernels (gs-voxelizer_amd/csrc/gsv_numerics.h)."""
import math

import numpy as np
import pytest

import oracle as O


def _ulp(x):
    return float(np.spacing(np.float32(abs(x)))) if x != 0 else float(np.spacing(np.float32(0)))


def test_logf_matches_math_log_within_2ulp():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        (2.0 ** rng.uniform(-149, 128, 20000)).astype(np.float32),      # whole binary32 range
        rng.uniform(0.5, 2.0, 20000).astype(np.float32),                # around 1 (small logs)
        rng.uniform(0.0, 1e-6, 2000).astype(np.float32),                 # the opacity cut-off
        np.float32(2.0) ** np.arange(-149, 128, dtype=np.float32),      # exact powers of two
        np.array([1.4142135, 1.4142136, 0.70710677, 0.7071068, 1e6, 89.999, 90.0171],
                 dtype=np.float32),
    ])
    xs = xs[np.isfinite(xs) & (xs > 0)]
    worst = 0.0
    for x in xs[::7]:
        got = O.logf(float(x))
        ref = math.log(float(x))
        err = abs(got - ref) / _ulp(ref) if ref != 0 else abs(got)
        worst = max(worst, err)
    assert worst <= 2.0, worst


@pytest.mark.parametrize("x,expect", [(0.0, -math.inf), (-0.0, -math.inf), (1.0, 0.0),
                                      (math.inf, math.inf)])
def test_logf_special_values(x, expect):
    assert O.logf(x) == expect


@pytest.mark.parametrize("x", [-1.0, -1e-30, -math.inf, math.nan])
def test_logf_nan_domain(x):
    assert math.isnan(O.logf(x))


@pytest.mark.parametrize("x,expect", [(0.9, 0), (-0.9, 0), (-1.5, -1), (7.99, 7), (8.0, 8),
                                      (math.nan, 0), (3e9, 2147483647), (-3e9, -2147483648),
                                      (math.inf, 2147483647), (-math.inf, -2147483648)])
def test_f2i_saturating_truncation(x, expect):
    assert O.f2i_sat(x) == expect
