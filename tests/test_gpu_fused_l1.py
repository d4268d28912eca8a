"""The voxelizer fused with the L1 loss of the reference's training loop
(README.md:77-82) against the unfused drop-in path: torch's l1_loss on the
volume voxelize_gaussians returns.  The fused backward forms torch's own
dL/dvolume, sgn(volume - target) * grad / numel, so every gradient must match
bit for bit; the loss matches to float summation order."""
import pytest
import torch
import torch.nn.functional as F

from gs_voxelizer import optim_to_render, synthetic as S, voxelize
from helpers import small_config

pytestmark = pytest.mark.gpu


def _leaves(work, device):
    w = work.to(device)
    return [t.clone().requires_grad_() for t in (w.pos3d, w.scale3d, w.quat, w.intensities)]


def _project(work, leaves):
    cfg = work.cfg
    pos3d, scale3d, quat, inten = leaves
    return optim_to_render.optim_to_render(pos3d, scale3d, quat, inten, cfg.vol, cfg.world,
                                           cfg.center)


def _unfused(work, device, target, extra=None, per_gaussian=True):
    leaves = _leaves(work, device)
    pr, cn, tmin, tmax, nt = _project(work, leaves)
    vol = voxelize.voxelize_gaussians(pr, cn, leaves[3], work.cfg.vol, tmin, tmax, nt,
                                      use_per_gaussian_backward=per_gaussian)
    tgt = target if target.dim() == 4 else target[..., None]
    loss = F.l1_loss(vol, tgt.expand_as(vol))
    total = loss if extra is None else loss + (vol * extra).sum()
    total.backward()
    return loss.detach(), vol.detach(), [l.grad for l in leaves]


def _fused(work, device, target, extra=None, per_gaussian=True):
    leaves = _leaves(work, device)
    pr, cn, tmin, tmax, nt = _project(work, leaves)
    loss, vol = voxelize.voxelize_gaussians_l1_loss(pr, cn, leaves[3], work.cfg.vol, tmin, tmax,
                                                    nt, target,
                                                    use_per_gaussian_backward=per_gaussian)
    total = loss if extra is None else loss + (vol * extra).sum()
    total.backward()
    return loss.detach(), vol.detach(), [l.grad for l in leaves]


def _scenes():
    yield "cfg1", S.make_gaussians(S.CONFIGS[1], seed=0)
    yield "multichannel_c3", S.make_gaussians(
        small_config(1, 3000, channels=3, world=(1.0, 1.5, 0.8), center=(0.5, 0.7, 0.5)), seed=3)
    yield "cfg2_10k", S.make_gaussians(small_config(2, 10000), seed=2)


@pytest.mark.parametrize("per_gaussian", [True, False])
@pytest.mark.parametrize("name,work", list(_scenes()), ids=lambda v: v if isinstance(v, str) else "")
def test_fused_l1_matches_unfused_bitwise(device, name, work, per_gaussian):
    cfg = work.cfg
    C = work.intensities.shape[1]
    target = S.phantom(work, device=device)
    if C > 1:
        g = torch.Generator(device="cpu").manual_seed(4)
        target = torch.rand(cfg.vol + (C,), generator=g).to(device)
    ref_loss, ref_vol, ref_grads = _unfused(work, device, target, per_gaussian=per_gaussian)
    loss, vol, grads = _fused(work, device, target, per_gaussian=per_gaussian)
    assert torch.equal(vol, ref_vol), name
    assert float(loss) == pytest.approx(float(ref_loss), rel=1e-6)
    for nm, a, b in zip(("pos3d", "scale3d", "quat", "intensity"), grads, ref_grads):
        assert torch.equal(a, b), f"{name}: grad {nm}"


def test_fused_l1_adds_the_volume_gradient(device):
    """A volume also used elsewhere: that gradient joins the fused one."""
    work = S.make_gaussians(small_config(1, 2000), seed=5)
    target = S.phantom(work, device=device)
    g = torch.Generator(device="cpu").manual_seed(6)
    extra = (torch.randn(work.cfg.vol + (1,), generator=g) * 1e-7).to(device)
    _, _, ref_grads = _unfused(work, device, target, extra=extra)
    _, _, grads = _fused(work, device, target, extra=extra)
    for a, b in zip(grads, ref_grads):
        assert torch.equal(a, b)


def test_fused_l1_no_intersections(device):
    """Every Gaussian outside the volume: loss = mean |target|, zero gradients."""
    work = S.make_gaussians(small_config(1, 64, vol=(16, 16, 16)), seed=7)
    work.pos3d += 10.0
    target = S.phantom(work, device=device)
    loss, vol, grads = _fused(work, device, target)
    assert float(vol.abs().sum()) == 0.0
    assert float(loss) == pytest.approx(float(target.abs().mean()), rel=1e-6)
    for g in grads:
        assert float(g.abs().sum()) == 0.0


@pytest.mark.parametrize("per_gaussian", [True, False])
def test_fused_l1_nan_and_inf_targets_match_unfused(device, per_gaussian):
    """Target voxels that are NaN or +-inf, inside the Gaussians' support: torch's
    l1_loss backward passes grad * sign(NaN) = 0 at a NaN difference and
    grad * -+1 at an infinite one; the fused backward must give the same
    gradients bit for bit (the loss is NaN on both paths)."""
    work = S.make_gaussians(small_config(1, 2000), seed=8)
    target = S.phantom(work, device=device).clone()
    g = torch.Generator(device="cpu").manual_seed(9)
    flat = target.view(-1)
    idx = torch.randperm(flat.numel(), generator=g)[:600].to(device)
    flat[idx[:400]] = float("nan")
    flat[idx[400:500]] = float("inf")
    flat[idx[500:]] = float("-inf")
    ref_loss, ref_vol, ref_grads = _unfused(work, device, target, per_gaussian=per_gaussian)
    loss, vol, grads = _fused(work, device, target, per_gaussian=per_gaussian)
    assert torch.equal(vol, ref_vol)
    assert torch.isnan(ref_loss) and torch.isnan(loss)
    for nm, a, b in zip(("pos3d", "scale3d", "quat", "intensity"), grads, ref_grads):
        assert torch.isfinite(b).all(), nm
        assert torch.equal(a, b), f"grad {nm}"


def test_fused_l1_sign_bytes_keep_denormal_differences(device):
    """The stored sign bytes are torch's sign(volume - target) element for
    element, also where the difference is a denormal number (targets of
    +-1e-40 where the volume is 0).  The library's voxelize code runs in
    binary32 flush-to-zero mode,
    where a denormal operand reads as 0; the sign is decided on the bit
    patterns, as IEEE arithmetic with denormals (torch's) decides it."""
    import gs_voxelizer.cuda as _C
    from helpers import gpu_bin
    work = S.make_gaussians(small_config(1, 2000), seed=10)
    cfg, n = work.cfg, work.cfg.n
    w = work.to(device)
    pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(n, w.pos3d, w.scale3d, w.quat,
                                                        w.intensities, cfg.vol, cfg.world,
                                                        cfg.center)
    _, _, ids, bins = gpu_bin(n, tmin, tmax, nt, cfg.vol)
    vol0 = _C.voxelize_forward(cfg.vol, ids, bins, pr, cn, w.intensities).reshape(-1)
    target = S.phantom(work, device=device).clone().reshape(-1)
    g = torch.Generator(device="cpu").manual_seed(11)
    zero = torch.nonzero(vol0 == 0).view(-1).cpu()
    zi = zero[torch.randperm(zero.numel(), generator=g)[:400]].to(device)
    target[zi[:200]] = 1e-40
    target[zi[200:]] = -1e-40
    assert bool((target[zi].abs() < 1.2e-38).all()) and bool((target[zi] != 0).all())
    vol, loss, sign = _C.voxelize_forward_l1(cfg.vol, ids, bins, pr, cn, w.intensities,
                                             target.view(cfg.vol))
    assert torch.equal(vol.reshape(-1), vol0)
    ref = torch.sign(vol.reshape(-1) - target)
    assert torch.equal(ref[zi], -torch.sign(target[zi]))  # torch keeps the denormal difference
    assert torch.equal(sign.reshape(-1).to(torch.float32), ref)
