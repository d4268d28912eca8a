"""The oracle reproduces the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py) exactly: a regression pin on the
checker itself."""
import glob
import os

import numpy as np
import pytest

import oracle as O

FIXTURES = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_oracle_reproduces_golden(path):
    f = np.load(path)  # plain arrays, allow_pickle=False
    vol, world, center = tuple(int(v) for v in f["vol_size"]), tuple(f["world"]), tuple(f["center"])
    r = O.pipeline(f["pos3d"], f["scale3d"], f["quat"], f["intensities"], vol, world, center,
                   vol_grad=f["vol_grad"])
    for k in ("tile_min", "tile_max", "num_tiles_hit", "cum_tiles_hit", "gaussian_ids_sorted",
              "tile_bins"):
        np.testing.assert_array_equal(r[k], f[k], err_msg=k)
    for k in ("pos3d_radii", "conics", "volume", "dpos3d_radii", "dconics", "dintensities",
              "dpos3d", "dscale3d", "dquat"):
        np.testing.assert_array_equal(r[k], f[k], err_msg=k)


def test_fixtures_present():
    assert len(FIXTURES) >= 2
