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
