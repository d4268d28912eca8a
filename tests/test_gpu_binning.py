"""HIP prefix sum and binning against the oracle: bit-exact.

gaussian_ids_sorted and tile_bins must equal the stable (tile, gaussian)
order the reference's CUB sort produces; the oracle's counting sort gives
that order by construction (pinned by test_oracle_binning.py).
"""
import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import synthetic as S
from helpers import gpu_bin, np32, oracle_project, small_config

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 7, 2047, 2048, 2049, 100_000, 1_000_003])
def test_cumsum_matches_numpy(device, n):
    import gs_voxelizer.cuda as _C
    g = np.random.default_rng(n)
    x = g.integers(0, 300, size=n).astype(np.int32)
    x[g.random(n) < 0.3] = 0
    cum, total = _C.cumsum_tiles_hit(torch.from_numpy(x).to(device))
    ref = np.cumsum(x.astype(np.int64))
    np.testing.assert_array_equal(np32(cum), ref.astype(np.int32))
    assert int(total.item()) == int(ref[-1])


def _bin_cases():
    yield "cfg1", S.make_gaussians(S.CONFIGS[1], seed=0)
    yield "cfg2_full", S.make_gaussians(S.CONFIGS[2], seed=0)
    yield "cfg3_full", S.make_gaussians(S.CONFIGS[3], seed=0)
    # one tile (no radix pass), a few tiles (one pass), > 65536 tiles (three passes)
    yield "one_tile", S.make_gaussians(small_config(1, 500, vol=(5, 7, 6)), seed=4)
    yield "few_tiles", S.make_gaussians(small_config(1, 2000, vol=(20, 40, 33)), seed=5)
    yield "three_passes", S.make_gaussians(small_config(3, 30000, vol=(520, 520, 520)), seed=6)
    yield "clustered_heavy", S.make_gaussians(small_config(5, 40000), seed=7)


@pytest.mark.parametrize("name,work", list(_bin_cases()), ids=lambda v: v if isinstance(v, str) else "")
def test_binning_matches_oracle_bit_exact(device, name, work):
    cfg = work.cfg
    n = work.pos3d.shape[0]
    rpr, rcn, rtmin, rtmax, rnt = oracle_project(work)
    rcum = O.cumsum(rnt)
    rI = int(rcum[-1])
    rids, rbins = O.bin_and_sort(n, rI, rtmin, rtmax, rcum, cfg.vol)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    cum, I, ids, bins = gpu_bin(n, t(rtmin), t(rtmax), t(rnt), cfg.vol)
    torch.cuda.synchronize()
    assert I == rI, (name, I, rI)
    np.testing.assert_array_equal(np32(cum), rcum, err_msg=f"{name}: cum_tiles_hit")
    np.testing.assert_array_equal(np32(bins), rbins, err_msg=f"{name}: tile_bins")
    np.testing.assert_array_equal(np32(ids), rids, err_msg=f"{name}: gaussian_ids_sorted")


def test_binning_empty(device):
    import gs_voxelizer.cuda as _C
    z = torch.zeros((3, 3), dtype=torch.int32, device=device)
    cum = torch.zeros((3,), dtype=torch.int32, device=device)
    ids, bins = _C.bin_and_sort_gaussians(3, 0, z, z, cum, (16, 16, 24))
    torch.cuda.synchronize()
    assert ids.numel() == 0
    assert bins.shape == (2 * 2 * 3, 2) and int(bins.abs().sum()) == 0
