"""The drop-in Python API end to end, as the reference's README example and
test/test_gs_voxelizer.py drive it: optim_to_render -> voxelize_gaussians ->
loss.backward(), leaf gradients compared with the oracle pipeline."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from gs_voxelizer import optim_to_render, synthetic as S, voxelize
from helpers import l1_vol_grad, np32, report_close, small_config

pytestmark = pytest.mark.gpu


def _run_api(work, device, per_gaussian=True, target=None, buffer=False):
    cfg = work.cfg
    w = work.to(device)
    leaves = [t.clone().requires_grad_() for t in (w.pos3d, w.scale3d, w.quat, w.intensities)]
    pos3d, scale3d, quat, inten = leaves
    buf = torch.empty((pos3d.shape[0], 4), device=device) if buffer else None
    pr, cn, tmin, tmax, nt = optim_to_render.optim_to_render(
        pos3d, scale3d, quat, inten, cfg.vol, cfg.world, cfg.center, pos3d_radii_buffer=buf)
    vol = voxelize.voxelize_gaussians(pr, cn, inten, cfg.vol, tmin, tmax, nt,
                                      use_per_gaussian_backward=per_gaussian)
    if target is None:
        target = S.phantom(work, device=device)
    tgt = target[..., None].expand_as(vol)
    loss = F.l1_loss(vol, tgt)
    loss.backward()
    torch.cuda.synchronize()
    return vol.detach(), [l.grad for l in leaves], target


@pytest.mark.parametrize("case", ["cfg1", "multichannel_c2", "cfg2_10k"])
@pytest.mark.parametrize("per_gaussian", [True, False])
def test_api_matches_oracle_pipeline(device, case, per_gaussian):
    if case == "cfg1":
        work = S.make_gaussians(S.CONFIGS[1], seed=0)
    elif case == "multichannel_c2":
        work = S.make_gaussians(small_config(1, 5000, channels=2, world=(1.0, 1.5, 0.8),
                                             center=(0.5, 0.7, 0.5)), seed=1)
    else:
        work = S.make_gaussians(small_config(2, 10000), seed=2)
    vol, grads, target = _run_api(work, device, per_gaussian)
    cfg = work.cfg
    ref_fwd = O.pipeline(work.pos3d.numpy(), work.scale3d.numpy(), work.quat.numpy(),
                         work.intensities.numpy(), cfg.vol, cfg.world, cfg.center)
    _, amb = O.voxelize_fwd(cfg.vol, ref_fwd["gaussian_ids_sorted"], ref_fwd["tile_bins"],
                            ref_fwd["pos3d_radii"], ref_fwd["conics"], work.intensities.numpy(),
                            with_amb=True)
    # gate-ambiguous terms (alpha*mean within 1e-4 of the threshold) may differ
    report_close(f"{case}: volume", np32(vol), ref_fwd["volume"], 1e-4, 1e-6, bound=amb)
    tgt = np.broadcast_to(target.cpu().numpy()[..., None], ref_fwd["volume"].shape)
    g = l1_vol_grad(np32(vol), tgt)  # same sign pattern the GPU loss saw
    ref = O.pipeline(work.pos3d.numpy(), work.scale3d.numpy(), work.quat.numpy(),
                     work.intensities.numpy(), cfg.vol, cfg.world, cfg.center, vol_grad=g)
    for nm, got, key in zip(("pos3d", "scale3d", "quat", "intensity"), grads,
                            ("dpos3d", "dscale3d", "dquat", "dintensities")):
        assert torch.isfinite(got).all(), nm
        report_close(f"{case}: grad {nm}", np32(got), ref[key], 1e-4, 1e-6)


def test_api_pos3d_radii_buffer(device):
    work = S.make_gaussians(small_config(1, 1000), seed=3)
    cfg = work.cfg
    w = work.to(device)
    buf = torch.full((1000, 4), -1.0, device=device)
    pr, *_ = optim_to_render.optim_to_render(w.pos3d, w.scale3d, w.quat, w.intensities,
                                             cfg.vol, cfg.world, cfg.center, pos3d_radii_buffer=buf)
    assert pr.data_ptr() == buf.data_ptr()
    rpr = O.project_fwd(work.pos3d.numpy(), work.scale3d.numpy(), work.quat.numpy(),
                        work.intensities.numpy(), cfg.vol, cfg.world, cfg.center)[0]
    np.testing.assert_array_equal(np32(buf), rpr)
    with pytest.raises(ValueError):
        optim_to_render.optim_to_render(w.pos3d, w.scale3d, w.quat, w.intensities, cfg.vol,
                                        cfg.world, cfg.center,
                                        pos3d_radii_buffer=torch.empty((999, 4), device=device))


def test_api_all_culled_gives_zero_volume_and_grads(device):
    cfg = small_config(1, 64, vol=(16, 16, 16))
    work = S.make_gaussians(cfg, seed=4)
    work.pos3d += 10.0  # every Gaussian far outside the volume -> num_intersects == 0
    vol, grads, _ = _run_api(work, device)
    assert vol.shape == (16, 16, 16, 1) and float(vol.abs().sum()) == 0.0
    for g in grads:
        assert float(g.abs().sum()) == 0.0


def test_api_zero_gaussians_in_voxelize(device):
    vol = voxelize.voxelize_gaussians(
        torch.zeros((0, 4), device=device), torch.zeros((0, 6), device=device),
        torch.zeros((0, 1), device=device), (8, 9, 10),
        torch.zeros((0, 3), dtype=torch.int32, device=device),
        torch.zeros((0, 3), dtype=torch.int32, device=device),
        torch.zeros((0,), dtype=torch.int32, device=device))
    assert vol.shape == (8, 9, 10, 1) and float(vol.abs().sum()) == 0.0


def test_api_channel_limit_and_device_checks(device):
    import gs_voxelizer.cuda as _C
    w = S.make_gaussians(small_config(1, 10), seed=5).to(device)
    with pytest.raises(RuntimeError, match="MAX_CHANNELS"):
        _C.optim_to_render_forward(10, w.pos3d, w.scale3d, w.quat, torch.ones((10, 5), device=device),
                                   (8, 8, 8), (1.0, 1.0, 1.0), (0.5, 0.5, 0.5))
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        _C.optim_to_render_forward(10, w.pos3d.cpu(), w.scale3d, w.quat, w.intensities,
                                   (8, 8, 8), (1.0, 1.0, 1.0), (0.5, 0.5, 0.5))


def test_speculative_capacity_matches_host_count(device, monkeypatch):
    """Forwards after the first launch binning at a recorded capacity without
    reading the count on the host.  Through a capacity overflow (a larger scene),
    a speculative hit and a shrink (a much smaller scene), volumes and gradients
    equal those of the reference's host-read path bit for bit."""
    scenes = [S.make_gaussians(small_config(1, 800), seed=21),
              S.make_gaussians(small_config(1, 6000), seed=22),   # more pairs: overflow
              S.make_gaussians(small_config(1, 6000), seed=22),   # same again: speculative hit
              S.make_gaussians(small_config(1, 40), seed=23)]     # far fewer: shrink
    voxelize._capacity.clear()
    spec = []
    for work in scenes:
        spec.append(_run_api(work, device, target=torch.zeros(work.cfg.vol, device=device)))
    caps = dict(voxelize._capacity)
    monkeypatch.setenv("GSV_SYNC_COUNT", "1")
    for work, (vol_s, grads_s, _) in zip(scenes, spec):
        vol, grads, _ = _run_api(work, device, target=torch.zeros(work.cfg.vol, device=device))
        assert torch.equal(vol, vol_s)
        for a, b in zip(grads, grads_s):
            assert torch.equal(a, b)
    assert len(caps) == 1 and 0 < next(iter(caps.values())) < 40 * 400
