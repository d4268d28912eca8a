"""BASELINE configurations 4 and 5 at their full sizes (1M Gaussians on 512^3 with
30.6M pairs; 500k clustered Gaussians, 4 channels, with 118M pairs).

- projection and binning: bit-exact against the oracle, every element, through
  both sort paths;
- forward: every voxel of the whole volume against the oracle (rel 1e-4 /
  abs 1e-6 plus the gate-ambiguous mass), and no less accurate than the
  oracle against the binary64 truth (helpers.assert_no_less_accurate);
- backward: every element of dpos3d_radii, dconics and dintensities for a
  whole-volume N(0,1) vol_grad, no less accurate than the oracle against the
  binary64 truth;
- backward: the size-independent identity sum_g I_gc dL/dI_gc == sum_v vol_vc g_vc
  per channel (the volume is linear in each channel's intensities once the gate,
  which depends on the mean intensity, is fixed), with finiteness of every
  gradient; and the same bits when the backward takes the forward's cull flags
  as its work list (chained rows off).
"""
import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import synthetic as S
from helpers import AccuracyChecks, assert_no_less_accurate, np32, oracle_project, report_close

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
    # the voxelize inputs are the same bits on both sides
    np.testing.assert_array_equal(np32(pr).view(np.uint32), rpr.view(np.uint32))
    np.testing.assert_array_equal(np32(cn).view(np.uint32), rcn.view(np.uint32))
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


def test_whole_volume_every_voxel(full):
    import gs_voxelizer.cuda as _C
    P = full
    work = P["work"]
    cfg = work.cfg
    vol = np32(_C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"],
                                   P["w"].intensities))
    args = (cfg.vol, np32(P["ids"]), np32(P["bins"]), P["rpr"], P["rcn"], work.intensities.numpy())
    print(f"{cfg.name}: oracle forward (binary32, binary64)", flush=True)
    ref, amb = O.voxelize_fwd(*args, with_amb=True)
    report_close(f"{cfg.name} whole volume", vol, ref, RTOL, ATOL, bound=amb)
    del amb
    truth, tamb = O.f64.voxelize_fwd(*args, with_amb=True)
    assert_no_less_accurate(f"{cfg.name} whole volume vs binary64", vol, ref, truth, tamb)


def test_every_gradient_element_whole_volume(full):
    """vol_grad N(0,1) over the whole volume; every element of the three
    gradients, per-pair reduction with the binning's tiles; the per-voxel form
    path (chained rows off) under the strict tier."""
    import gs_voxelizer.cuda as _C
    P = full
    work = P["work"]
    cfg = work.cfg
    C = work.intensities.shape[1]
    g = np.random.default_rng(23).standard_normal(cfg.vol + (C,)).astype(np.float32)
    def device(chains):
        before = _C.set_backward_chains(chains)
        try:
            return [np32(t) for t in _C.voxelize_backward_per_gaussian(
                cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], P["w"].intensities,
                torch.from_numpy(g).to(P["pr"].device), P["tmin"], P["tmax"], P["cum"],
                tiles_sorted=P["tiles"])]
        finally:
            _C.set_backward_chains(before)
    got, form = device(True), device(False)
    args = (cfg.vol, np32(P["ids"]), np32(P["bins"]), P["rpr"], P["rcn"], work.intensities.numpy(),
            g)
    print(f"{cfg.name}: oracle backward (binary32)", flush=True)
    ref = O.voxelize_bwd(*args)
    # the binary64 truth in four tile ranges (its per-pair diagnostics of a
    # whole cfg5 volume would take ~37 GB at once); each Gaussian's sums over
    # the ranges add up in binary64
    T = np32(P["bins"]).shape[0]
    truth = [np.zeros(a.shape, np.float64) for a in ref]
    tamb = [np.zeros(a.shape, np.float64) for a in ref]
    for k in range(4):
        print(f"{cfg.name}: oracle backward (binary64), tiles {k}/4", flush=True)
        tg, _, am = O.f64.voxelize_bwd(*args, tile_range=(k * T // 4, (k + 1) * T // 4),
                                       diagnostics=True)
        for acc, part in zip(truth + tamb, list(tg) + list(am)):
            acc += part
    checks = AccuracyChecks()
    for nm, a, f, b, t, m in zip(("dpos3d_radii", "dconics", "dintensities"), got, form, ref,
                                 truth, tamb):
        checks.check(f"{cfg.name} whole-volume normal: {nm}", a, b, t, m)
        checks.check(f"{cfg.name} whole-volume normal, form rows: {nm}", f, b, t, m, strict=True)
    checks.done()
