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


# 5M and 20M elements: more than 2048 blocks of 2048, so the block sums are
# scanned by their own workgroup (in one tile of 8192, then in several)
@pytest.mark.parametrize("n", [1, 7, 2047, 2048, 2049, 100_000, 1_000_003, 5_000_011, 20_000_003])
def test_cumsum_matches_numpy(device, n):
    import gs_voxelizer.cuda as _C
    g = np.random.default_rng(n)
    x = g.integers(0, 300 if n < 2_000_000 else 50, size=n).astype(np.int32)  # total < 2^31
    x[g.random(n) < 0.3] = 0
    cum, total = _C.cumsum_tiles_hit(torch.from_numpy(x).to(device))
    ref = np.cumsum(x.astype(np.int64))
    np.testing.assert_array_equal(np32(cum), ref.astype(np.int32))
    assert int(total.item()) == int(ref[-1])


def _bin_cases():
    yield "cfg1", S.make_gaussians(S.CONFIGS[1], seed=0)
    yield "cfg2_full", S.make_gaussians(S.CONFIGS[2], seed=0)
    yield "cfg3_full", S.make_gaussians(S.CONFIGS[3], seed=0)
    # one tile (no radix pass), a few tiles (one pass), 17- and 18-bit tile ids
    # (two 9-bit passes), 19 bits (three 8-bit passes)
    yield "one_tile", S.make_gaussians(small_config(1, 500, vol=(5, 7, 6)), seed=4)
    yield "few_tiles", S.make_gaussians(small_config(1, 2000, vol=(20, 40, 33)), seed=5)
    yield "bits17", S.make_gaussians(small_config(3, 20000, vol=(400, 408, 320)), seed=9)
    yield "bits18", S.make_gaussians(small_config(3, 30000, vol=(512, 512, 512)), seed=10)
    yield "three_passes", S.make_gaussians(small_config(3, 30000, vol=(520, 520, 520)), seed=6)
    yield "clustered_heavy", S.make_gaussians(small_config(5, 40000), seed=7)
    # extreme aspect ratios: 375 tiles along x (9 padded x bits, 8 buckets of
    # 512 keys), 375 tile layers along z with 2 tiles per row, and 625 tiles
    # along x (10 x bits: the bucket path steps aside for the LSD passes)
    yield "wide_x", S.make_gaussians(small_config(3, 20000, vol=(16, 24, 3000)), seed=12)
    yield "tall_z", S.make_gaussians(small_config(3, 20000, vol=(3000, 24, 16)), seed=13)
    yield "wider_x", S.make_gaussians(small_config(3, 8000, vol=(8, 8, 5000)), seed=14)


@pytest.mark.parametrize("name,work", list(_bin_cases()), ids=lambda v: v if isinstance(v, str) else "")
def test_binning_matches_oracle_bit_exact(device, binning_path, name, work):
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


def test_binning_empty(device, binning_path):
    import gs_voxelizer.cuda as _C
    z = torch.zeros((3, 3), dtype=torch.int32, device=device)
    cum = torch.zeros((3,), dtype=torch.int32, device=device)
    ids, bins = _C.bin_and_sort_gaussians(3, 0, z, z, cum, (16, 16, 24))
    torch.cuda.synchronize()
    assert ids.numel() == 0
    assert bins.shape == (2 * 2 * 3, 2) and int(bins.abs().sum()) == 0


def _emission(tmin, tmax, Tx, Ty):
    """Keys and Gaussian ids in emission order: Gaussian-major, each box's tiles
    z -> y -> x (bin_and_sort_gaussians.cu:11-35)."""
    keys, vals = [], []
    for g in range(tmin.shape[0]):
        (x0, y0, z0), (x1, y1, z1) = tmin[g], tmax[g]
        if x1 <= x0 or y1 <= y0 or z1 <= z0:
            continue
        z, y, x = np.meshgrid(np.arange(z0, z1), np.arange(y0, y1), np.arange(x0, x1),
                              indexing="ij")
        keys.append(((z * Ty + y) * Tx + x).ravel())
        vals.append(np.full(keys[-1].size, g))
    if not keys:
        return np.zeros(0, np.int64), np.zeros(0, np.int64)
    return np.concatenate(keys), np.concatenate(vals)


def _device_count_bin(device, n, tmin, tmax, nt, vol, capacity):
    import gs_voxelizer.cuda as _C
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    cum, total = _C.cumsum_tiles_hit(t(nt))
    ids, bins = _C.bin_and_sort_gaussians_device_count(n, capacity, total, t(tmin), t(tmax), cum,
                                                       vol)
    torch.cuda.synchronize()
    return int(total.item()), np32(ids), np32(bins)


@pytest.mark.parametrize("name,work", [c for c in _bin_cases() if c[0] in
                                       ("cfg1", "few_tiles", "three_passes", "clustered_heavy")],
                         ids=lambda v: v if isinstance(v, str) else "")
def test_device_count_binning_matches_host_count(device, binning_path, name, work):
    """The count read on the device, capacity above it: same bits as the oracle."""
    cfg = work.cfg
    n = work.pos3d.shape[0]
    _, _, rtmin, rtmax, rnt = oracle_project(work)
    rcum = O.cumsum(rnt)
    rI = int(rcum[-1])
    rids, rbins = O.bin_and_sort(n, rI, rtmin, rtmax, rcum, cfg.vol)
    I, ids, bins = _device_count_bin(device, n, rtmin, rtmax, rnt, cfg.vol, rI + 5000)
    assert I == rI
    np.testing.assert_array_equal(bins, rbins)
    np.testing.assert_array_equal(ids[:rI], rids)


def test_device_count_binning_over_capacity_sorts_the_prefix(device, binning_path):
    """Capacity below the count: exactly the first `capacity` emitted pairs are
    sorted (stable by tile), and the call neither fails nor writes past it."""
    work = S.make_gaussians(small_config(1, 3000, vol=(40, 48, 56)), seed=3)
    cfg = work.cfg
    n = work.pos3d.shape[0]
    _, _, rtmin, rtmax, rnt = oracle_project(work)
    Tx, Ty, Tz = O.tile_grid(cfg.vol)
    keys, vals = _emission(rtmin, rtmax, Tx, Ty)
    cap = keys.size // 2 + 17
    order = np.argsort(keys[:cap], kind="stable")
    I, ids, bins = _device_count_bin(device, n, rtmin, rtmax, rnt, cfg.vol, cap)
    assert I == keys.size and ids.shape == (cap,)
    np.testing.assert_array_equal(ids, vals[:cap][order])
    counts = np.bincount(keys[:cap], minlength=Tx * Ty * Tz)
    np.testing.assert_array_equal(bins[:, 1] - bins[:, 0], counts)


def test_binning_long_runs_of_empty_gaussians(device, binning_path):
    """Runs of 5000 Gaussians without tiles between large boxes: chunks whose
    Gaussians lie beyond the emission block's cached window of cum."""
    import gs_voxelizer.cuda as _C
    vol = (160, 160, 160)
    Tx, Ty, Tz = O.tile_grid(vol)
    n = 20000
    rng = np.random.default_rng(11)
    tmin = np.zeros((n, 3), np.int32)
    tmax = np.zeros((n, 3), np.int32)
    for g in range(0, n, 5000):
        lo = rng.integers(0, 6, 3)
        tmin[g] = lo
        tmax[g] = lo + rng.integers(8, 14, 3)
    nt = np.prod(np.maximum(tmax - tmin, 0), axis=1).astype(np.int32)
    cum = O.cumsum(nt)
    rI = int(cum[-1])
    rids, rbins = O.bin_and_sort(n, rI, tmin, tmax, cum, vol)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    ids, bins = _C.bin_and_sort_gaussians(n, rI, t(tmin), t(tmax), t(cum), vol)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(np32(bins), rbins)
    np.testing.assert_array_equal(np32(ids), rids)
    I2, ids2, bins2 = _device_count_bin(device, n, tmin, tmax, nt, vol, rI)
    np.testing.assert_array_equal(bins2, rbins)
    np.testing.assert_array_equal(ids2, rids)


def _fused_bin(device, n, tmin, tmax, nt, vol, capacity):
    import gs_voxelizer.cuda as _C
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    host = torch.full((1,), -1, dtype=torch.int64).pin_memory()
    cum, total, ids, bins, tiles = _C.cumsum_bin_and_sort_device_count(
        n, capacity, t(nt), t(tmin), t(tmax), vol, total_host=host, return_tiles=True)
    torch.cuda.synchronize()
    assert int(host.item()) == int(total.item())
    return np32(cum), int(total.item()), np32(ids), np32(bins), np32(tiles)


@pytest.mark.parametrize("name,work", [c for c in _bin_cases() if c[0] in
                                       ("cfg1", "cfg2_full", "cfg3_full", "one_tile", "few_tiles",
                                        "bits17", "bits18", "clustered_heavy", "wide_x", "tall_z",
                                        "wider_x")],
                         ids=lambda v: v if isinstance(v, str) else "")
def test_fused_cumsum_binning_matches_oracle(device, binning_path, name, work):
    """gsv_cumsum_bin_and_sort_device_count (the bucket counts and their prefix
    formed beside the scan's two passes) gives the oracle's prefix sum, count,
    ids, bins and sorted tiles bit for bit, on both sort paths."""
    cfg = work.cfg
    n = work.pos3d.shape[0]
    _, _, rtmin, rtmax, rnt = oracle_project(work)
    rcum = O.cumsum(rnt)
    rI = int(rcum[-1])
    rids, rbins = O.bin_and_sort(n, rI, rtmin, rtmax, rcum, cfg.vol)
    rtiles = np.repeat(np.arange(rbins.shape[0]), rbins[:, 1] - rbins[:, 0])
    cum, I, ids, bins, tiles = _fused_bin(device, n, rtmin, rtmax, rnt, cfg.vol, rI + 3000)
    assert I == rI, (name, I, rI)
    np.testing.assert_array_equal(cum, rcum, err_msg=f"{name}: cum_tiles_hit")
    np.testing.assert_array_equal(bins, rbins, err_msg=f"{name}: tile_bins")
    np.testing.assert_array_equal(ids[:rI], rids, err_msg=f"{name}: gaussian_ids_sorted")
    np.testing.assert_array_equal(tiles[:rI], rtiles, err_msg=f"{name}: tiles_sorted")


def test_fused_cumsum_binning_empty_and_over_capacity(device, binning_path):
    """No Gaussians: a zero count and zeroed bins.  Capacity below the count:
    the call returns, reports the full count, and a second call at that count
    bins exactly (what voxelize.py does)."""
    cum, I, ids, bins, tiles = _fused_bin(device, 0, np.zeros((0, 3), np.int32),
                                          np.zeros((0, 3), np.int32), np.zeros(0, np.int32),
                                          (16, 16, 24), 100)
    assert I == 0 and cum.size == 0 and int(np.abs(bins).sum()) == 0
    work = S.make_gaussians(small_config(1, 3000, vol=(40, 48, 56)), seed=3)
    cfg = work.cfg
    n = work.pos3d.shape[0]
    _, _, rtmin, rtmax, rnt = oracle_project(work)
    rcum = O.cumsum(rnt)
    rI = int(rcum[-1])
    rids, rbins = O.bin_and_sort(n, rI, rtmin, rtmax, rcum, cfg.vol)
    cum, I, ids, bins, _ = _fused_bin(device, n, rtmin, rtmax, rnt, cfg.vol, rI // 2 + 17)
    assert I == rI and ids.shape == (rI // 2 + 17,)
    np.testing.assert_array_equal(cum, rcum)
    cum, I, ids, bins, _ = _fused_bin(device, n, rtmin, rtmax, rnt, cfg.vol, rI)
    np.testing.assert_array_equal(bins, rbins)
    np.testing.assert_array_equal(ids, rids)
