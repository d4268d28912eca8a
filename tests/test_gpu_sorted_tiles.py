"""The binning's sorted keys handed to the backward, and the pair count written
straight into pinned host memory.

- tiles_sorted from bin_and_sort_gaussians(..., return_tiles=True) is exactly the
  tile of each sorted pair, i.e. tile t repeated over tile_bins[t];
- the backward given tiles_sorted gives the same bits as the one that rebuilds
  the pair -> tile map itself;
- sparse scenes, where most 64-pair backward waves span more tiles than one wave
  stages (3 for one channel, 2 otherwise), still match the oracle: those pairs
  are found and processed by the second backward kernel;
- cumsum_tiles_hit(total_host=...) leaves the count in pinned memory.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import synthetic as S
from helpers import l1_vol_grad, np32, oracle_project, report_close, small_config

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-6


def _cases():
    yield "cfg1", S.make_gaussians(S.CONFIGS[1], seed=0)
    yield "edge_tiles", S.make_gaussians(small_config(1, 800, vol=(20, 30, 17)), seed=8)
    yield "sparse_c1", S.make_gaussians(small_config(1, 600, vol=(64, 72, 56)), seed=3)
    yield "sparse_c3", S.make_gaussians(small_config(1, 500, vol=(64, 64, 64), channels=3), seed=4)


def _project(work, device):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    w = work.to(device)
    n = w.pos3d.shape[0]
    pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(n, w.pos3d, w.scale3d, w.quat,
                                                        w.intensities, cfg.vol, cfg.world,
                                                        cfg.center)
    return w, n, pr, cn, tmin, tmax, nt


def _tiles_from_bins(bins, I):
    b = np32(bins).astype(np.int64)
    out = np.full(I, -1, np.int64)
    for t in np.nonzero(b[:, 1] > b[:, 0])[0]:
        out[b[t, 0]:b[t, 1]] = t
    return out


@pytest.mark.parametrize("name,work", list(_cases()), ids=lambda v: v if isinstance(v, str) else "")
def test_tiles_sorted_is_the_tile_of_each_sorted_pair(device, binning_path, name, work):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    w, n, pr, cn, tmin, tmax, nt = _project(work, device)
    cum, total = _C.cumsum_tiles_hit(nt)
    I = int(total.item())
    ids, bins = _C.bin_and_sort_gaussians(n, I, tmin, tmax, cum, cfg.vol)
    ids2, bins2, tiles = _C.bin_and_sort_gaussians(n, I, tmin, tmax, cum, cfg.vol,
                                                   return_tiles=True)
    assert torch.equal(ids, ids2) and torch.equal(bins, bins2)
    np.testing.assert_array_equal(np32(tiles).astype(np.int64), _tiles_from_bins(bins, I))
    cap = I + 1000
    ids3, bins3, tiles3 = _C.bin_and_sort_gaussians_device_count(
        n, cap, total, tmin, tmax, cum, cfg.vol, return_tiles=True)
    assert torch.equal(ids3[:I], ids) and torch.equal(bins3, bins)
    assert torch.equal(tiles3[:I], tiles)


@pytest.mark.parametrize("name,work", list(_cases()), ids=lambda v: v if isinstance(v, str) else "")
def test_backward_with_sorted_tiles_matches_oracle_and_rebuilt_map(device, name, work):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    w, n, pr, cn, tmin, tmax, nt = _project(work, device)
    cum, total = _C.cumsum_tiles_hit(nt)
    I = int(total.item())
    ids, bins, tiles = _C.bin_and_sort_gaussians(n, I, tmin, tmax, cum, cfg.vol,
                                                 return_tiles=True)
    # how many backward waves span more tiles than one wave stages
    K = 3 if w.intensities.shape[1] == 1 else 2
    t = np32(tiles)
    spans = [len(np.unique(t[p:p + 64])) for p in range(0, I, 64)]
    if name.startswith("sparse"):
        assert sum(s > K for s in spans) > len(spans) // 2, spans[:20]
    vol = _C.voxelize_forward(cfg.vol, ids, bins, pr, cn, w.intensities)
    target = S.phantom(work).numpy()[..., None]
    g = l1_vol_grad(np32(vol), np.broadcast_to(target, tuple(vol.shape)))
    gd = torch.from_numpy(g).to(device)
    got = _C.voxelize_backward_per_gaussian(cfg.vol, ids, bins, pr, cn, w.intensities, gd, tmin,
                                            tmax, cum, tiles_sorted=tiles)
    rebuilt = _C.voxelize_backward_per_gaussian(cfg.vol, ids, bins, pr, cn, w.intensities, gd,
                                                tmin, tmax, cum)
    for a, b in zip(got, rebuilt):
        assert torch.equal(a, b)
    rpr, rcn, rtmin, rtmax, rnt = oracle_project(work)
    rcum = O.cumsum(rnt)
    rids, rbins = O.bin_and_sort(n, int(rcum[-1]), rtmin, rtmax, rcum, cfg.vol)
    ref, absum, amb = O.voxelize_bwd(cfg.vol, rids, rbins, rpr, rcn, work.intensities.numpy(), g,
                                     diagnostics=True)
    for nm, a, b, s, m in zip(("dpos3d_radii", "dconics", "dintensities"), got, ref, absum, amb):
        report_close(f"{name}: {nm}", np32(a), b, RTOL, ATOL, bound=1e-5 * s + m)


def test_cumsum_total_in_pinned_memory(device):
    import gs_voxelizer.cuda as _C
    rng = np.random.default_rng(0)
    for n in (1, 2047, 2049, 300_000):
        x = rng.integers(0, 50, n).astype(np.int32)
        host = torch.full((1,), -7, dtype=torch.int64, pin_memory=True)
        cum, total = _C.cumsum_tiles_hit(torch.from_numpy(x).to(device), total_host=host)
        ev = torch.cuda.Event()
        ev.record()
        ev.synchronize()
        assert int(host[0]) == int(x.astype(np.int64).sum()) == int(total.item())
    with pytest.raises(RuntimeError):
        _C.cumsum_tiles_hit(torch.zeros(4, dtype=torch.int32, device=device),
                            total_host=torch.zeros(1, dtype=torch.int64))
