"""Shared helpers for the parity tests: run the HIP path and the CPU oracle on
the same seeded inputs and compare them."""
import os

import numpy as np
import torch

import oracle as O
from gs_voxelizer import synthetic as S


def small_config(base: int, n: int, vol=None, channels=None, world=None, center=None, **kw):
    """A reduced variant of benchmark config `base` (same distributions)."""
    c = S.CONFIGS[base]
    d = dict(name=f"{c.name}_n{n}", vol=vol or c.vol, n=n, channels=channels or c.channels,
             scale=c.scale, quat=c.quat, intensity=c.intensity, position=c.position,
             phantom=c.phantom, world=world or c.world, center=center or c.center)
    d.update(kw)
    return S.Config(**d)


def np32(t):
    return t.detach().cpu().numpy()


def gpu_project(work, device):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    w = work.to(device)
    return _C.optim_to_render_forward(cfg.n if w.pos3d.shape[0] == cfg.n else w.pos3d.shape[0],
                                      w.pos3d, w.scale3d, w.quat, w.intensities, cfg.vol,
                                      cfg.world, cfg.center)


def oracle_project(work):
    cfg = work.cfg
    return O.project_fwd(work.pos3d.numpy(), work.scale3d.numpy(), work.quat.numpy(),
                         work.intensities.numpy(), cfg.vol, cfg.world, cfg.center)


def gpu_bin(n, tmin, tmax, nt, vol):
    import gs_voxelizer.cuda as _C
    cum, total = _C.cumsum_tiles_hit(nt)
    I = int(total.item())
    ids, bins = _C.bin_and_sort_gaussians(n, I, tmin, tmax, cum, vol)
    return cum, I, ids, bins


def report_close(name, got, ref, rtol, atol, bound=None, log_only=False):
    """assert |got-ref| <= atol + rtol*|ref| (+ bound, an optional per-element
    allowance such as a summation-error bound) elementwise; message lists the worst.
    With log_only the comparison is only logged (GSV_MARGIN_LOG), not asserted."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    allow = atol + rtol * np.abs(ref)
    if bound is not None:
        allow = allow + np.asarray(bound, dtype=np.float64)
    err = np.abs(got - ref)
    bad = ~(err <= allow)  # NaN counts as bad unless both NaN
    both_nan = np.isnan(got) & np.isnan(ref)
    bad &= ~both_nan
    log = os.environ.get("GSV_MARGIN_LOG")
    if log and err.size:
        # how close parity runs: the worst fraction of the whole allowance used,
        # of the plain atol + rtol*|ref| alone, and how many elements needed the
        # extra per-element bound (gate ambiguity, conditioning) at all
        plain = atol + rtol * np.abs(ref)
        with np.errstate(divide="ignore", invalid="ignore"):
            used = np.where(both_nan, 0.0, err / allow)
            used_plain = np.where(both_nan, 0.0, err / plain)
        beyond = int(((err > plain) & ~both_nan).sum())
        with open(log, "a") as f:
            f.write(f"{name}\t{err.size}\t{beyond}\t{float(np.nanmax(used)):.4g}\t"
                    f"{float(np.nanmax(used_plain)):.4g}\n")
    if bad.any() and not log_only:
        idx = np.argsort(-(err - allow).ravel())[:5]
        worst = [(np.unravel_index(i, got.shape), got.ravel()[i], ref.ravel()[i]) for i in idx]
        raise AssertionError(f"{name}: {int(bad.sum())}/{bad.size} elements outside "
                             f"rtol={rtol} atol={atol}; worst {worst}")


def l1_vol_grad(vol, target):
    """Gradient of mean |vol - target| w.r.t. vol (torch.nn.functional.l1_loss)."""
    return (np.sign(vol.astype(np.float64) - target.astype(np.float64)) / vol.size).astype(np.float32)
