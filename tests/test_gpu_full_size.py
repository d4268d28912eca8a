"""BASELINE configurations 4 and 5 at their full sizes (1M Gaussians on 512^3 with
30.6M pairs; 500k clustered Gaussians, 4 channels, with 118M pairs).

- projection and binning: bit-exact against the oracle, every element;
- forward: every voxel of the first z-layer of tiles, and of the z-layer that
  holds the heaviest tile (cfg5: a cluster centre, ~11.5k pairs), against the
  oracle;
- backward on the heaviest layer: vol_grad N(0,1) there and zero elsewhere,
  so only that layer's tiles contribute, and every element of the three
  gradients against the oracle restricted to those tiles;
- backward: the size-independent identity sum_g I_gc dL/dI_gc == sum_v vol_vc g_vc
  per channel (the volume is linear in each channel's intensities once the gate,
  which depends on the mean intensity, is fixed), with finiteness of every
  gradient; and the same bits when the backward takes the forward's cull flags
  as its work list.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import synthetic as S
from helpers import np32, oracle_project, report_close

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-6


def _full(device, c):
    import gs_voxelizer.cuda as _C
    work = S.make_gaussians(S.CONFIGS[c], seed=0)
    cfg = work.cfg
    n = cfg.n
    w = work.to(device)
    pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(n, w.pos3d, w.scale3d, w.quat,
                                                        w.intensities, cfg.vol, cfg.world,
                                                        cfg.center)
    rpr, rcn, rtmin, rtmax, rnt = oracle_project(work)
    np.testing.assert_array_equal(np32(tmin), rtmin)
    np.testing.assert_array_equal(np32(tmax), rtmax)
    np.testing.assert_array_equal(np32(nt), rnt)
    cum, total = _C.cumsum_tiles_hit(nt)
    I = int(total.item())
    ids, bins, tiles = _C.bin_and_sort_gaussians(n, I, tmin, tmax, cum, cfg.vol, return_tiles=True)
    return dict(work=work, w=w, pr=pr, cn=cn, tmin=tmin, tmax=tmax, cum=cum, I=I, ids=ids,
                bins=bins, tiles=tiles, rpr=rpr, rcn=rcn, rtmin=rtmin, rtmax=rtmax, rnt=rnt)


@pytest.fixture(scope="module", params=[4, 5], ids=["cfg4_512cube_1M", "cfg5_clustered_c4"])
def full(request, device):
    P = _full(device, request.param)
    yield P
    del P
    torch.cuda.empty_cache()


def test_binning_bit_exact(full):
    P = full
    cfg = P["work"].cfg
    rcum = O.cumsum(P["rnt"])
    rI = int(rcum[-1])
    assert P["I"] == rI
    rids, rbins = O.bin_and_sort(cfg.n, rI, P["rtmin"], P["rtmax"], rcum, cfg.vol)
    np.testing.assert_array_equal(np32(P["cum"]), rcum)
    np.testing.assert_array_equal(np32(P["bins"]), rbins)
    np.testing.assert_array_equal(np32(P["ids"]), rids)
    counts = rbins[:, 1] - rbins[:, 0]
    np.testing.assert_array_equal(np.bincount(np32(P["tiles"]), minlength=counts.size), counts)


@pytest.mark.parametrize("path", ["lsd", "bucket"])
def test_binning_each_path_same_bits(full, path, monkeypatch):
    """Both sort paths at full size (cfg5 through the bucket path: buckets of
    ~460k pairs, far beyond the LDS staging) give the bits checked above."""
    import gs_voxelizer.cuda as _C
    P = full
    cfg = P["work"].cfg
    monkeypatch.setenv("GSV_BINNING", path)
    ids, bins, tiles = _C.bin_and_sort_gaussians(cfg.n, P["I"], P["tmin"], P["tmax"], P["cum"],
                                                 cfg.vol, return_tiles=True)
    assert torch.equal(bins, P["bins"])
    assert torch.equal(ids, P["ids"])
    assert torch.equal(tiles, P["tiles"])


def test_forward_first_tile_layer(full):
    import gs_voxelizer.cuda as _C
    P = full
    work = P["work"]
    cfg = work.cfg
    vol = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], P["w"].intensities)
    Tx, Ty, _ = O.tile_grid(cfg.vol)
    ref, amb = O.voxelize_fwd(cfg.vol, np32(P["ids"]), np32(P["bins"]), P["rpr"], P["rcn"],
                              work.intensities.numpy(), tile_range=(0, Tx * Ty), with_amb=True)
    report_close(f"{cfg.name} first tile layer", np32(vol[:8]), ref[:8], RTOL, ATOL,
                 bound=amb[:8])
    assert float(vol[8:].abs().sum()) > 0


def test_backward_intensity_identity(full, set_chains):
    import gs_voxelizer.cuda as _C
    P = full
    cfg = P["work"].cfg
    inten = P["w"].intensities
    vol = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], inten)
    gen = torch.Generator(device="cpu").manual_seed(7)
    g = torch.randn(vol.shape, generator=gen).to(vol.device)
    dp, dc, di = _C.voxelize_backward_per_gaussian(cfg.vol, P["ids"], P["bins"], P["pr"],
                                                   P["cn"], inten, g, P["tmin"], P["tmax"],
                                                   P["cum"], tiles_sorted=P["tiles"])
    for c in range(inten.shape[1]):
        lhs = float((inten[:, c].double() * di[:, c].double()).sum())
        prod = vol[..., c].double() * g[..., c].double()
        rhs, scale = float(prod.sum()), float(prod.abs().sum())
        assert abs(lhs - rhs) <= 1e-5 * scale, (c, lhs, rhs, scale)
    for t in (dp, dc, di):
        assert torch.isfinite(t).all()
    assert float(dp[:, 3].abs().sum()) == 0.0
    # the forward's cull flags as the backward's work list (more than 2048
    # blocks of flags here: the counts are scanned by one workgroup first)
    live = torch.empty(P["I"], device=inten.device, dtype=torch.uint8)
    vol2 = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], inten,
                               pair_live=live)
    assert torch.equal(vol2, vol)
    assert P["I"] > 2048 * 4096
    bwd = lambda **kw: _C.voxelize_backward_per_gaussian(cfg.vol, P["ids"], P["bins"], P["pr"],
                                                         P["cn"], inten, g, P["tmin"], P["tmax"],
                                                         P["cum"], tiles_sorted=P["tiles"], **kw)
    # the flags change which pairs share a wave, and a group takes the chained
    # rows only when all of its pairs qualify: equal to rounding with them on,
    # bit for bit without them
    # (elementwise the gap follows each sum's cancellation against N(0,1)
    # vol_grad, which the oracle comparisons bound; here the whole arrays)
    for a, b in zip((dp, dc, di), bwd(pair_live=live)):
        gap = float(torch.linalg.vector_norm((a - b).double()))
        assert gap <= 1e-4 * float(torch.linalg.vector_norm(a.double())), (cfg.name, gap)
    set_chains(False)
    for a, b in zip(bwd(), bwd(pair_live=live)):
        assert torch.equal(a, b)


def _heaviest_layer(P):
    cfg = P["work"].cfg
    bins = np32(P["bins"])
    counts = bins[:, 1] - bins[:, 0]
    Tx, Ty, _ = O.tile_grid(cfg.vol)
    t = int(np.argmax(counts))
    z = t // (Tx * Ty)
    return z, (z * Tx * Ty, (z + 1) * Tx * Ty), int(counts[t])


def test_forward_heaviest_tile_layer(full):
    import gs_voxelizer.cuda as _C
    P = full
    work = P["work"]
    cfg = work.cfg
    z, rng, heaviest = _heaviest_layer(P)
    print(f"{cfg.name}: heaviest tile has {heaviest} pairs, tile layer {z}", flush=True)
    vol = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], P["w"].intensities)
    ref, amb = O.voxelize_fwd(cfg.vol, np32(P["ids"]), np32(P["bins"]), P["rpr"], P["rcn"],
                              work.intensities.numpy(), tile_range=rng, with_amb=True)
    zs = slice(8 * z, 8 * z + 8)
    report_close(f"{cfg.name} heaviest tile layer {z} ({heaviest} pairs)", np32(vol[zs]),
                 ref[zs], RTOL, ATOL, bound=amb[zs])


def test_backward_heaviest_tile_layer_every_element(full):
    """vol_grad is N(0,1) on the heaviest tile layer and exactly zero elsewhere:
    every other tile's terms are then exactly zero, so the whole-volume GPU
    backward equals the oracle's over that layer's tiles."""
    import gs_voxelizer.cuda as _C
    P = full
    work = P["work"]
    cfg = work.cfg
    C = work.intensities.shape[1]
    z, rng, heaviest = _heaviest_layer(P)
    g = np.zeros(cfg.vol + (C,), np.float32)
    zs = slice(8 * z, min(8 * z + 8, cfg.vol[0]))
    g[zs] = np.random.default_rng(23).standard_normal(g[zs].shape).astype(np.float32)
    got = _C.voxelize_backward_per_gaussian(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"],
                                            P["w"].intensities, torch.from_numpy(g).to(
                                                P["pr"].device), P["tmin"], P["tmax"],
                                            P["cum"], tiles_sorted=P["tiles"])
    torch.cuda.synchronize()
    rg, absum, amb = O.voxelize_bwd(cfg.vol, np32(P["ids"]), np32(P["bins"]), P["rpr"],
                                    P["rcn"], work.intensities.numpy(), g, tile_range=rng,
                                    diagnostics=True)
    for nm, a, b, s, m in zip(("dpos3d_radii", "dconics", "dintensities"), got, rg, absum, amb):
        report_close(f"{cfg.name} heaviest layer {z}: {nm}", np32(a), b, RTOL, ATOL,
                     bound=1e-5 * s + m)
