"""Tile culling by a separating axis, and the backward's work list built from it.

The forward skips a (tile, Gaussian) pair when a separating-axis test proves
that no point of the tile's voxel-centre box lies in the Gaussian's gate
ellipsoid, and reports its decision per sorted pair (pair_live).  Checked here:

- conservative: every voxel centre of every culled pair's tile fails the
  reference's gates (sigma <= 0 and exp(sigma) * mean >= 1e-6), evaluated in
  binary64 from the kernel's own inputs; on scenes with needle-shaped Gaussians
  too, whose conics are far from isotropic;
- effective: a good share of the pairs of a scene of rotated anisotropic
  Gaussians is culled (isotropic ones leave few: their 3-sigma boxes barely
  reach beyond the gate ellipsoid);
- the backward given the flags (evaluating only the kept pairs, zero partials
  for the culled ones) returns the same bits as without them, for vol_grad and
  fused-L1 sources, in host-count and capacity (device-count) modes, including
  sparse scenes whose waves span more tiles than one wave stages.  That holds
  with the backward's chained rows off (set_backward_chains(False)): with them on, a
  group of pairs takes them only when all of its pairs qualify, and the flags
  change which pairs share a wave, so there the two agree to rounding
  (rel 1e-4 / abs 1e-6) instead;
- the backward depends on no stale workspace contents: a workspace of 0x00
  bytes and one of 0xFF bytes give the same bits, with and without the work
  list.
"""
import dataclasses

import numpy as np
import pytest
import torch

from gs_voxelizer import synthetic as S
from helpers import l1_vol_grad, np32, report_close, small_config

pytestmark = pytest.mark.gpu


def _needles(base_cfg, n, seed):
    """Uniform scene of thin rotated needles: one axis 2-8 voxels, two 0.1-0.4."""
    work = S.make_gaussians(small_config(base_cfg, n, vol=(48, 56, 40)), seed=seed)
    g = torch.Generator().manual_seed(seed + 100)
    cfg = work.cfg
    vs = torch.tensor([cfg.world[2] / cfg.vol[2], cfg.world[1] / cfg.vol[1],
                       cfg.world[0] / cfg.vol[0]])  # (x, y, z) voxel sizes
    lo, hi = np.log(0.1), np.log(0.4)
    s = torch.exp(lo + (hi - lo) * torch.rand(n, 3, generator=g))
    long_axis = torch.randint(0, 3, (n,), generator=g)
    s[torch.arange(n), long_axis] = torch.exp(np.log(2.0) + (np.log(8.0) - np.log(2.0)) *
                                             torch.rand(n, generator=g))
    return dataclasses.replace(work, scale3d=(s * vs).to(torch.float32))


def _cases():
    yield "cfg1", S.make_gaussians(S.CONFIGS[1], seed=0)
    yield "cfg2_small", S.make_gaussians(small_config(2, 8000, vol=(64, 64, 64)), seed=1)
    yield "edge_tiles", S.make_gaussians(small_config(1, 800, vol=(20, 30, 17)), seed=8)
    yield "sparse_c1", S.make_gaussians(small_config(1, 600, vol=(64, 72, 56)), seed=3)
    yield "sparse_c3", S.make_gaussians(small_config(1, 500, vol=(64, 64, 64), channels=3),
                                        seed=4)
    yield "needles", _needles(1, 3000, seed=6)


CASES = list(_cases())
IDS = [c[0] for c in CASES]


def _run(work, device):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    w = work.to(device)
    n = w.pos3d.shape[0]
    pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(n, w.pos3d, w.scale3d, w.quat,
                                                        w.intensities, cfg.vol, cfg.world,
                                                        cfg.center)
    cum, total = _C.cumsum_tiles_hit(nt)
    I = int(total.item())
    ids, bins, tiles = _C.bin_and_sort_gaussians(n, I, tmin, tmax, cum, cfg.vol,
                                                 return_tiles=True)
    live = torch.full((I,), 7, device=device, dtype=torch.uint8)
    vol = _C.voxelize_forward(cfg.vol, ids, bins, pr, cn, w.intensities, pair_live=live)
    return dict(w=w, n=n, pr=pr, cn=cn, tmin=tmin, tmax=tmax, nt=nt, cum=cum, total=total, I=I,
                ids=ids, bins=bins, tiles=tiles, live=live, vol=vol)


def _passing(cfg, pr, cn, inten, g, tile):
    """Whether any inside voxel centre of `tile` passes Gaussian g's gates (binary64)."""
    D, H, W = cfg.vol
    Tx, Ty = (W + 7) // 8, (H + 7) // 8
    tx, ty, tz = tile % Tx, (tile // Tx) % Ty, tile // (Tx * Ty)
    xs = np.arange(tx * 8, min(tx * 8 + 8, W)) + 0.5
    ys = np.arange(ty * 8, min(ty * 8 + 8, H)) + 0.5
    zs = np.arange(tz * 8, min(tz * 8 + 8, D)) + 0.5
    Z, Y, X = np.meshgrid(zs, ys, xs, indexing="ij")
    dx, dy, dz = pr[g, 0] - X, pr[g, 1] - Y, pr[g, 2] - Z
    a, b, c, d, e, f = cn[g]
    sig = -0.5 * (a * dx * dx + d * dy * dy + f * dz * dz) - (b * dx * dy + c * dx * dz +
                                                              e * dy * dz)
    mean = inten[g].mean()
    with np.errstate(over="ignore", invalid="ignore"):
        ok = np.isfinite(sig) & (sig <= 0) & (np.exp(sig) * mean >= 1e-6)
    return bool(ok.any())


@pytest.mark.parametrize("name,work", CASES, ids=IDS)
def test_culled_pairs_have_no_passing_voxel(device, name, work):
    R = _run(work, device)
    flags = np32(R["live"])
    assert set(np.unique(flags)) <= {0, 1}  # every pair of every tile range was flagged
    pr = np32(R["pr"]).astype(np.float64)
    cn = np32(R["cn"]).astype(np.float64)
    inten = work.intensities.numpy().astype(np.float64)
    ids, tiles = np32(R["ids"]), np32(R["tiles"])
    culled = np.nonzero(flags == 0)[0]
    for p in culled:
        assert not _passing(work.cfg, pr, cn, inten, int(ids[p]), int(tiles[p])), (name, p)
    if name in ("cfg1", "needles"):  # anisotropic, rotated: many box corners miss the gate
        assert culled.size > 0.03 * R["I"], (name, culled.size, R["I"])


def _agree(what, a, b, exact):
    if exact:
        assert torch.equal(a, b), what
    else:
        report_close(what, np32(a), np32(b), 1e-4, 1e-6)


@pytest.mark.parametrize("chain", ["0", "1"], ids=["chain_off", "chain_on"])
@pytest.mark.parametrize("name,work", CASES, ids=IDS)
def test_backward_with_cull_flags_is_bitwise_equal(device, set_chains, name, work, chain):
    import gs_voxelizer.cuda as _C
    set_chains(chain == "1")
    exact = chain == "0"
    R = _run(work, device)
    cfg, w = work.cfg, R["w"]
    args = (cfg.vol, R["ids"], R["bins"], R["pr"], R["cn"], w.intensities)
    boxes = (R["tmin"], R["tmax"], R["cum"])
    target = S.phantom(work).numpy()[..., None]
    g = l1_vol_grad(np32(R["vol"]), np.broadcast_to(target, tuple(R["vol"].shape)))
    gd = torch.from_numpy(g).to(device)
    plain = _C.voxelize_backward_per_gaussian(*args, gd, *boxes, tiles_sorted=R["tiles"])
    culled = _C.voxelize_backward_per_gaussian(*args, gd, *boxes, tiles_sorted=R["tiles"],
                                               pair_live=R["live"])
    for a, b in zip(plain, culled):
        _agree(f"{name} vol_grad", a, b, exact)
    # fused L1 source
    tgt = torch.from_numpy(np.ascontiguousarray(np.broadcast_to(target, tuple(R["vol"].shape))))
    vol, loss, sign = _C.voxelize_forward_l1(*args, tgt.to(device).float())
    gl = torch.full((1,), 0.75, device=device)
    plain = _C.voxelize_backward_l1(*args, sign, gl, None, *boxes, tiles_sorted=R["tiles"])
    culled = _C.voxelize_backward_l1(*args, sign, gl, None, *boxes, tiles_sorted=R["tiles"],
                                     pair_live=R["live"])
    for a, b in zip(plain, culled):
        _agree(f"{name} fused L1", a, b, exact)
    # capacity-sized arrays with the live count on the device
    cap = R["I"] + 777
    ids_c, bins_c, tiles_c = _C.bin_and_sort_gaussians_device_count(
        R["n"], cap, R["total"], R["tmin"], R["tmax"], R["cum"], cfg.vol, return_tiles=True)
    live_c = torch.full((cap,), 3, device=device, dtype=torch.uint8)
    _C.voxelize_forward(cfg.vol, ids_c, bins_c, R["pr"], R["cn"], w.intensities,
                        pair_live=live_c)
    assert torch.equal(live_c[:R["I"]], R["live"])
    got = _C.voxelize_backward_per_gaussian(cfg.vol, ids_c, bins_c, R["pr"], R["cn"],
                                            w.intensities, gd, *boxes, tiles_sorted=tiles_c,
                                            count_dev=R["total"], pair_live=live_c)
    plain = _C.voxelize_backward_per_gaussian(*args, gd, *boxes, tiles_sorted=R["tiles"])
    for a, b in zip(plain, got):
        _agree(f"{name} capacity", a, b, exact)


def _bwd_on_workspace(R, cfg, gd, fill, with_flags):
    """Per-Gaussian backward through the C-ABI on a workspace of `fill` bytes."""
    import ctypes
    import gs_voxelizer.cuda as _C
    w, n, I = R["w"], R["n"], R["I"]
    D, H, W = cfg.vol
    C = _C._channels(w.intensities)
    nbytes = ctypes.c_size_t(0)
    _C._call("voxelize_bwd_workspace_bytes", D, H, W, C, n, I, 1, ctypes.byref(nbytes))
    ws = torch.full((nbytes.value,), fill, device=gd.device, dtype=torch.uint8)
    f32 = dict(device=gd.device, dtype=torch.float32)
    dpos, dconic, dint = (torch.empty((n, k), **f32) for k in (4, 6, C))
    null = ctypes.c_void_p(0)
    live = _C._ptr(R["live"]) if with_flags else null
    with torch.cuda.device(gd.device):
        _C._call("voxelize_bwd", D, H, W, C, n, I, _C._ptr(R["ids"]), _C._ptr(R["bins"]),
                 _C._ptr(R["pr"]), _C._ptr(R["cn"]), _C._ptr(w.intensities), _C._ptr(gd),
                 _C._ptr(R["tmin"]), _C._ptr(R["tmax"]), _C._ptr(R["cum"]),
                 _C._ptr(R["tiles"]), null, live, _C._ptr(dpos), _C._ptr(dconic), _C._ptr(dint),
                 1, _C._ptr(ws), nbytes.value, _C._stream(gd.device))
    torch.cuda.synchronize()
    return dpos, dconic, dint


@pytest.mark.parametrize("with_flags", [False, True], ids=["all_pairs", "work_list"])
@pytest.mark.parametrize("name,work", [c for c in CASES if c[0] in ("cfg1", "sparse_c1",
                                                                    "sparse_c3", "needles")],
                         ids=["cfg1", "sparse_c1", "sparse_c3", "needles"])
def test_backward_ignores_stale_workspace(device, name, work, with_flags):
    """The backward reads from its workspace only what the same call wrote there
    (the pair -> tile map, the partials, the work list and the per-wave flags
    that send waves spanning more than their staged tiles to the rest pass):
    gradients from a workspace of 0x00 bytes and of 0xFF bytes agree bitwise,
    on sparse scenes where many waves take the rest pass and on cfg1."""
    R = _run(work, device)
    cfg = work.cfg
    target = S.phantom(work).numpy()[..., None]
    g = l1_vol_grad(np32(R["vol"]), np.broadcast_to(target, tuple(R["vol"].shape)))
    gd = torch.from_numpy(np.ascontiguousarray(g)).to(device)
    zeros = _bwd_on_workspace(R, cfg, gd, 0x00, with_flags)
    ones = _bwd_on_workspace(R, cfg, gd, 0xFF, with_flags)
    for what, a, b in zip(("dpos3d_radii", "dconics", "dintensities"), zeros, ones):
        assert torch.equal(a, b), (name, what)
    ref = _C_api_backward(R, cfg, gd, with_flags)
    for what, a, b in zip(("dpos3d_radii", "dconics", "dintensities"), zeros, ref):
        assert torch.equal(a, b), (name, what, "against the Python entry")


def _C_api_backward(R, cfg, gd, with_flags):
    import gs_voxelizer.cuda as _C
    w = R["w"]
    return _C.voxelize_backward_per_gaussian(cfg.vol, R["ids"], R["bins"], R["pr"], R["cn"],
                                             w.intensities, gd, R["tmin"], R["tmax"], R["cum"],
                                             tiles_sorted=R["tiles"],
                                             pair_live=R["live"] if with_flags else None)


def test_very_thin_gaussians_are_not_culled_from_tiles_they_reach(device):
    """Conics with one diagonal entry of 1e38 (det >= 2^126, whose binary32
    reciprocal flushes to zero) and a mean intensity of 5e-6 (so the gate's
    K^2 stays below 3.4 and K^2 * 1e38 finite): each Gaussian's centre sits
    on a voxel-centre plane across its thin axis and 0.3 voxel below a tile
    face in a wide one, 0.8 voxel from the first voxel centre of the next
    tile, which passes its gates.  No pair whose tile holds a passing voxel
    may be culled, and the volume matches the oracle's (channel 0, intensity
    1, carries ~0.7 there; channel 1 is -0.99999, so the mean is 5e-6)."""
    import gs_voxelizer.cuda as _C
    import oracle as O
    vol = (24, 24, 24)
    big = 1e38
    # thin along z, along x, along y; centre 0.3 voxel below a tile face in
    # a wide axis, on a voxel-centre plane in the thin one
    pr = np.array([[7.7, 11.5, 3.5, 1.0], [3.5, 7.7, 11.5, 1.0], [11.5, 3.5, 7.7, 1.0]],
                  np.float32)
    cn = np.array([[1, 0, 0, 1, 0, big], [big, 0, 0, 1, 0, 1], [1, 0, 0, big, 0, 1]],
                  np.float32)
    inten = np.tile(np.array([[1.0, -0.99999]], np.float32), (3, 1))
    # boxes (x, y, z) of two tiles across the face plus the tile holding the centre
    tmin = np.array([[0, 1, 0], [0, 0, 1], [1, 0, 0]], np.int32)
    tmax = np.array([[2, 2, 1], [1, 2, 2], [2, 1, 2]], np.int32)
    nt = np.prod(tmax - tmin, 1).astype(np.int32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    cum, total = _C.cumsum_tiles_hit(dev(nt))
    I = int(total.item())
    ids, bins, tiles = _C.bin_and_sort_gaussians(3, I, dev(tmin), dev(tmax), cum, vol,
                                                 return_tiles=True)
    live = torch.full((I,), 7, device=device, dtype=torch.uint8)
    out = _C.voxelize_forward(vol, ids, bins, dev(pr), dev(cn), dev(inten), pair_live=live)
    torch.cuda.synchronize()
    flags, ids_np, tiles_np = np32(live), np32(ids), np32(tiles)
    cfg = type("Cfg", (), {"vol": vol})
    passing = [_passing(cfg, pr.astype(np.float64), cn.astype(np.float64),
                        inten.astype(np.float64), int(g), int(t))
               for g, t in zip(ids_np, tiles_np)]
    assert sum(passing) == 6, passing  # both tiles of every box hold a passing voxel
    for p, (ok, f) in enumerate(zip(passing, flags)):
        assert not (ok and f == 0), ("culled a reachable tile", p, int(ids_np[p]),
                                     int(tiles_np[p]))
    ref, amb = O.voxelize_fwd(vol, ids_np, np32(bins), pr, cn, inten, with_amb=True)
    report_close("very thin Gaussians: volume", np32(out), ref, 1e-4, 1e-6, bound=amb)
    assert ref[..., 0].max() > 0.3
