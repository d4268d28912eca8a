"""The reference's volume-scaling range (test/test_volume_scaling.py:30,
53-64, 130-139): cubic volumes of 1024 and 1200 voxels with 64,000 and 75,000
Gaussians of (0.03, 0.01, 0.02) world units (synthetic.volume_scaling_scenario),
through the public API under torch.inference_mode, as the reference runs them.

At 1024^3 the grid has 2^21 tiles, at 1200^3 3,375,000 (22-bit keys), so the
binning takes the LSD passes (three 8-bit passes; the bucket path serves keys
of up to 18 bits); the scenes have 187.8M and 345.7M (tile, Gaussian) pairs,
and the 1200^3 volume (1.73G voxels, 6.9 GB) puts element offsets past 2^31
bytes.  Checked against the oracle:

- tile boxes and counts bit-exact, the pair count, and the sorted ids and
  tile ranges of every pair bit-exact;
- the volume the public API returns, on the tile layer with the most pairs
  and on the last tile layer (the highest offsets): every voxel within rel
  1e-4 / abs 1e-6 (+ gate ambiguity) of the oracle, and no less accurate than
  it against the binary64 truth.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import optim_to_render, synthetic as S, voxelize
from helpers import assert_no_less_accurate, np32, report_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=[1024, 1200], ids=["edge1024_64k", "edge1200_75k"])
def scaled(request, device):
    work = S.volume_scaling_scenario(request.param, seed=0)
    cfg = work.cfg
    print(f"volume scaling {cfg.name}", flush=True)
    w = work.to(device)
    with torch.inference_mode():
        pr, cn, tmin, tmax, nt = optim_to_render.optim_to_render(
            w.pos3d, w.scale3d, w.quat, w.intensities, cfg.vol, cfg.world, cfg.center)
        vol = voxelize.voxelize_gaussians(pr, cn, w.intensities, cfg.vol, tmin, tmax, nt)
    torch.cuda.synchronize()
    assert tuple(vol.shape) == cfg.vol + (1,)
    rpr, rcn, rtmin, rtmax, rnt = O.project_fwd(work.pos3d.numpy(), work.scale3d.numpy(),
                                                work.quat.numpy(), work.intensities.numpy(),
                                                cfg.vol, cfg.world, cfg.center)
    np.testing.assert_array_equal(np32(tmin), rtmin)
    np.testing.assert_array_equal(np32(tmax), rtmax)
    np.testing.assert_array_equal(np32(nt), rnt)
    rcum = O.cumsum(rnt)
    I = int(rcum[-1])
    rids, rbins = O.bin_and_sort(cfg.n, I, rtmin, rtmax, rcum, cfg.vol)
    yield dict(work=work, w=w, vol=vol, pr=pr, cn=cn, tmin=tmin, tmax=tmax, nt=nt, rpr=rpr,
               rcn=rcn, rcum=rcum, I=I, rids=rids, rbins=rbins)
    del vol
    torch.cuda.empty_cache()


def test_binning_bit_exact_past_18_bit_keys(scaled):
    import gs_voxelizer.cuda as _C
    P = scaled
    cfg = P["work"].cfg
    Tx, Ty, Tz = O.tile_grid(cfg.vol)
    bits = int(np.ceil(np.log2(Tx * Ty * Tz)))
    assert bits == (21 if cfg.vol[0] == 1024 else 22)
    assert P["I"] == (187_770_590 if cfg.vol[0] == 1024 else 345_678_610)
    cum, total = _C.cumsum_tiles_hit(P["nt"])
    assert int(total.item()) == P["I"]
    np.testing.assert_array_equal(np32(cum), P["rcum"])
    ids, bins = _C.bin_and_sort_gaussians(cfg.n, P["I"], P["tmin"], P["tmax"], cum, cfg.vol)
    np.testing.assert_array_equal(np32(bins), P["rbins"])
    np.testing.assert_array_equal(np32(ids), P["rids"])


def _layers(P):
    bins = P["rbins"]
    cfg = P["work"].cfg
    Tx, Ty, Tz = O.tile_grid(cfg.vol)
    counts = (bins[:, 1] - bins[:, 0]).reshape(Tz, Ty * Tx).sum(1)
    return sorted({int(np.argmax(counts)), Tz - 1})


def test_forward_heaviest_and_last_tile_layers(scaled):
    P = scaled
    work = P["work"]
    cfg = work.cfg
    Tx, Ty, Tz = O.tile_grid(cfg.vol)
    D = cfg.vol[0]
    for z in _layers(P):
        zs = (8 * z, min(8 * z + 8, D))
        tiles = (z * Tx * Ty, (z + 1) * Tx * Ty)
        print(f"{cfg.name}: tile layer {z}", flush=True)
        got = np32(P["vol"][zs[0]:zs[1]])
        args = (cfg.vol, P["rids"], P["rbins"], P["rpr"], P["rcn"], work.intensities.numpy())
        ref, amb = O.voxelize_fwd(*args, tile_range=tiles, with_amb=True, z_slab=zs)
        report_close(f"{cfg.name} tile layer {z}", got, ref, 1e-4, 1e-6, bound=amb)
        truth, tamb = O.f64.voxelize_fwd(*args, tile_range=tiles, with_amb=True, z_slab=zs)
        assert_no_less_accurate(f"{cfg.name} tile layer {z} vs binary64", got, ref, truth, tamb)
        assert ref.max() > 0.1
