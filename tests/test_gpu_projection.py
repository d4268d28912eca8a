"""HIP projection (forward + backward) against the CPU oracle.

Bar: tile_min / tile_max / num_tiles_hit bit-exact (they decide binning);
float outputs within rel 1e-6 (both sides evaluate the same binary32
expressions without contraction, so they are expected to be identical).
"""
import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import synthetic as S
from helpers import np32, oracle_project, report_close, small_config

pytestmark = pytest.mark.gpu


def _cases():
    yield "cfg1", S.make_gaussians(S.CONFIGS[1], seed=0)
    for c in (2, 3, 4):
        # the reference's multi-channel scenario: non-cubic world, off-centre volume
        cfg = small_config(1, 3000, channels=c, world=(1.0, 1.5, 0.8), center=(0.5, 0.7, 0.5))
        yield f"multichannel_c{c}", S.make_gaussians(cfg, seed=c)
    yield "cfg2_iso_identity", S.make_gaussians(small_config(2, 20000), seed=1)
    yield "cfg5_heavy_tail_clustered", S.make_gaussians(small_config(5, 20000), seed=2)
    yield "cfg3_full", S.make_gaussians(S.CONFIGS[3], seed=0)


def _edge_work():
    """Hand-made rows: culled, degenerate, special extents, unnormalised quats."""
    cfg = small_config(1, 12, vol=(20, 30, 17))
    w = S.make_gaussians(cfg, seed=3)
    p, s, q, I = w.pos3d.clone(), w.scale3d.clone(), w.quat.clone(), w.intensities.clone()
    p[0] = torch.tensor([5.0, 5.0, 5.0])              # far outside -> culled
    s[1] = torch.tensor([0.0, 0.01, 0.01])             # det == 0 -> culled
    I[2] = 0.0                                         # log(0) -> extent 3 (fminf with NaN)
    I[3] = 5e-7                                        # mean*1e6 < 1 -> NaN extent -> 3
    I[4] = 2e-6                                        # extent = sqrt(2 ln 2) < 3
    I[5] = -0.3                                        # negative mean -> NaN -> 3
    q[6] = torch.tensor([2.0, 0.0, 0.0, 0.0])          # unnormalised identity
    q[7] = torch.tensor([0.7071068, 0.7071068, 0.0, 0.0])  # 90 degrees about x
    s[8] = torch.tensor([2.0, 2.0, 2.0])               # covers the whole volume
    p[9] = torch.tensor([-0.02, 0.5, 0.5])             # just outside, within radius
    s[10] = torch.tensor([1e-4, 1e-4, 1e-4])           # sub-voxel
    p[11] = torch.tensor([1.0, 1.0, 1.0])              # on the far corner
    return S.Workload(cfg, p, s, q, I, w.phantom_params)


@pytest.mark.parametrize("name,work", list(_cases()) + [("edge_rows", _edge_work())],
                         ids=lambda v: v if isinstance(v, str) else "")
def test_projection_forward_matches_oracle(device, name, work):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    w = work.to(device)
    out = _C.optim_to_render_forward(w.pos3d.shape[0], w.pos3d, w.scale3d, w.quat, w.intensities,
                                     cfg.vol, cfg.world, cfg.center)
    torch.cuda.synchronize()
    pr, cn, tmin, tmax, nt = (np32(t) for t in out)
    rpr, rcn, rtmin, rtmax, rnt = oracle_project(work)
    np.testing.assert_array_equal(tmin, rtmin, err_msg=f"{name}: tile_min")
    np.testing.assert_array_equal(tmax, rtmax, err_msg=f"{name}: tile_max")
    np.testing.assert_array_equal(nt, rnt, err_msg=f"{name}: num_tiles_hit")
    report_close(f"{name}: pos3d_radii", pr, rpr, rtol=1e-6, atol=0)
    report_close(f"{name}: conics", cn, rcn, rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("name,work", list(_cases())[:5] + [("edge_rows", _edge_work())],
                         ids=lambda v: v if isinstance(v, str) else "")
def test_projection_backward_matches_oracle(device, name, work):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    n = work.pos3d.shape[0]
    rpr, rcn, *_ = oracle_project(work)
    g = torch.Generator().manual_seed(11)
    dpr = torch.randn((n, 4), generator=g)
    dcn = torch.randn((n, 6), generator=g)
    w = work.to(device)
    dp, ds, dq = _C.optim_to_render_backward(n, w.pos3d, w.scale3d, w.quat, cfg.vol, cfg.world,
                                             cfg.center, dpr.to(device), dcn.to(device),
                                             torch.from_numpy(rpr).to(device))
    torch.cuda.synchronize()
    rdp, rds, rdq = O.project_bwd(work.pos3d.numpy(), work.scale3d.numpy(), work.quat.numpy(),
                                  cfg.vol, cfg.world, cfg.center, dpr.numpy(), dcn.numpy(), rpr)
    report_close(f"{name}: dpos3d", np32(dp), rdp, rtol=1e-6, atol=0)
    scale = max(1e-30, float(np.abs(rds).max()))
    report_close(f"{name}: dscale3d", np32(ds), rds, rtol=1e-5, atol=1e-6 * scale)
    scale = max(1e-30, float(np.abs(rdq).max()))
    report_close(f"{name}: dquat", np32(dq), rdq, rtol=1e-5, atol=1e-6 * scale)


@pytest.mark.parametrize("s_vox", [0.2, 0.45])
def test_projection_backward_regulariser_closed_form(device, s_vox):
    """The HIP projection backward against the closed form of the 1e-7 det^2
    regulariser (optim_to_render.cu:200) for identity-quaternion Gaussians that
    are isotropic in voxel units, one conic diagonal gradient per row, on
    non-cubic voxels: dscale_k = -2 s^9 g / ((s^12 + 1e-7) vs_k)."""
    import gs_voxelizer.cuda as _C
    vol, world, center = (40, 56, 48), (1.0, 1.5, 0.8), (0.5, 0.7, 0.5)
    vs = np.array([world[2] / vol[2], world[1] / vol[1], world[0] / vol[0]])
    pix = np.array([[19.3, 21.7, 13.4], [27.6, 9.2, 30.1], [5.3, 37.8, 22.9]])
    lo = np.array([center[2] - world[2] / 2, center[1] - world[1] / 2, center[0] - world[0] / 2])
    pos = torch.from_numpy((lo + pix * vs).astype(np.float32))
    scale = torch.from_numpy(np.tile((s_vox * vs).astype(np.float32), (3, 1)))
    quat = torch.tensor([[1.0, 0, 0, 0]] * 3)
    inten = torch.full((3, 1), 0.5)
    dev = [t.to(device) for t in (pos, scale, quat, inten)]
    pr, *_ = _C.optim_to_render_forward(3, *dev, vol, world, center)
    g = (1.5, -0.7, 2.0)
    dcn = torch.zeros((3, 6))
    dcn[0, 0], dcn[1, 3], dcn[2, 5] = g
    dp, ds, dq = _C.optim_to_render_backward(3, dev[0], dev[1], dev[2], vol, world, center,
                                             torch.zeros((3, 4), device=device),
                                             dcn.to(device), pr)
    torch.cuda.synchronize()
    s_eff = scale.numpy().astype(np.float64) / vs
    want = np.zeros((3, 3))
    for r, k in enumerate(range(3)):
        want[r, k] = -2.0 * s_eff[r, k] ** 9 * g[r] / ((s_eff[r, k] ** 12 + 1e-7) * vs[k])
    report_close(f"dscale closed form s={s_vox}", np32(ds), want, rtol=1e-4,
                 atol=1e-6 * np.abs(want).max())
    assert np.abs(np32(dq)).max() <= 1e-6 * np.abs(want).max()


def test_num_points_beyond_the_rows_is_refused(device):
    """A num_points larger than the per-Gaussian tensors is refused before any
    launch (the kernels would index past the tensors), in projection forward
    and backward and in binning; the GPU is not touched by the refused calls."""
    import gs_voxelizer.cuda as _C
    work = S.make_gaussians(small_config(1, 64, vol=(16, 16, 16)), seed=2)
    w = work.to(device)
    cfg = work.cfg
    n = w.pos3d.shape[0]
    with pytest.raises(RuntimeError, match="num_points"):
        _C.optim_to_render_forward(n + 1, w.pos3d, w.scale3d, w.quat, w.intensities, cfg.vol,
                                   cfg.world, cfg.center)
    pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(n, w.pos3d, w.scale3d, w.quat,
                                                        w.intensities, cfg.vol, cfg.world,
                                                        cfg.center)
    with pytest.raises(RuntimeError, match="num_points"):
        _C.optim_to_render_backward(n + 1, w.pos3d, w.scale3d, w.quat, cfg.vol, cfg.world,
                                    cfg.center, torch.zeros_like(pr), torch.zeros_like(cn), pr)
    cum, total = _C.cumsum_tiles_hit(nt)
    I = int(total.item())
    with pytest.raises(RuntimeError, match="num_points"):
        _C.bin_and_sort_gaussians(n + 1, I, tmin, tmax, cum, cfg.vol)
    with pytest.raises(RuntimeError, match="num_points"):
        _C.bin_and_sort_gaussians_device_count(n + 1, I, total, tmin, tmax, cum, cfg.vol)
    with pytest.raises(RuntimeError, match="non-negative"):
        _C.bin_and_sort_gaussians(-1, I, tmin, tmax, cum, cfg.vol)
    ids, bins = _C.bin_and_sort_gaussians(n, I, tmin, tmax, cum, cfg.vol)
    torch.cuda.synchronize()
    assert ids.numel() == I
