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


def accuracy(got, truth, allow_extra=None, rtol=1e-4, atol=1e-6):
    """(count, worst) of `got` against a binary64 `truth`: how many elements lie
    outside atol + rtol*|truth| (+ allow_extra, the gate-ambiguous mass), and the
    largest |got - truth| / that bound (NaN against a non-NaN counts as outside
    and as an infinite error)."""
    got = np.asarray(got, dtype=np.float64)
    truth = np.asarray(truth, dtype=np.float64)
    assert got.shape == truth.shape, (got.shape, truth.shape)
    allow = atol + rtol * np.abs(truth)
    if allow_extra is not None:
        allow = allow + np.asarray(allow_extra, dtype=np.float64)
    both_nan = np.isnan(got) & np.isnan(truth)
    with np.errstate(invalid="ignore"):
        err = np.where(both_nan, 0.0, np.abs(got - truth))
    err = np.where(np.isnan(err), np.inf, err)
    ratio = err / allow
    return int((ratio > 1.0).sum()), float(ratio.max()) if ratio.size else 0.0


def normalised_error_percentiles(got, truth, allow_extra, rtol, atol, qs):
    """Percentiles `qs` of |got - truth| / (atol + rtol*|truth| + allow_extra)."""
    got = np.asarray(got, dtype=np.float64)
    truth = np.asarray(truth, dtype=np.float64)
    allow = atol + rtol * np.abs(truth)
    if allow_extra is not None:
        allow = allow + np.asarray(allow_extra, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        r = np.abs(got - truth) / allow
    r = np.where(np.isnan(r), np.inf, r)
    return np.percentile(r, qs) if r.size else np.zeros(len(qs))


# How much less accurate than the binary32 oracle the device may be, per
# comparison against the binary64 truth, where an element's normalised error
# is |x - truth| / (atol + rtol*|truth| + allow_extra) and "outside" means
# above 1:
#   - elements outside: at most COUNT_SLACK_REL * the oracle's + COUNT_SLACK_ABS;
#   - 99.9th percentile of the normalised error: at most P999_FACTOR * the
#     oracle's, or 0.1;
#   - worst normalised error: at most WORST_FACTOR * the oracle's, or 1.
# Two tiers.  The default backward evaluates most rows as chained products (an
# anchor exp2 stepped along the row), whose exponent roundings (a per-row
# slope of up to ~40, an anchor up to 3 columns from the voxels it serves)
# are shared by several voxels and so average out of the gradient sums less
# than the oracle's per-voxel roundings: measured (cfg3, cfg5's 100k sample,
# N(0,1) vol_grad) it leaves ~0.3-2.5x the oracle's count of elements outside
# the bound, the most on cfg5's dpos and dintensities, and up to ~1.7x its
# 99.9th percentile.  With the chained rows off (GSV_BWD_CHAIN=0 or
# gsv_set_backward_chains(0): every row from the per-voxel form) the device is
# at or below the oracle's count in every such comparison, and STRICT holds.
COUNT_SLACK_REL, COUNT_SLACK_ABS, P999_FACTOR, WORST_FACTOR = 3.0, 10, 2.0, 4.0
STRICT = dict(count_rel=1.25, count_abs=10, p999=1.5, worst=2.0)


def assert_no_less_accurate(name, got, oracle32, truth, allow_extra=None, rtol=1e-4, atol=1e-6,
                            strict=False):
    """The device result `got` is no less accurate than the binary32 oracle's
    `oracle32` against the binary64 `truth` (each within atol + rtol*|truth| +
    allow_extra per element), up to the slack above (STRICT's with `strict`).
    The statistics are logged
    (GSV_MARGIN_LOG: name, elements, device count, oracle count, device worst,
    oracle worst, then the 99th, 99.9th and 99.99th percentiles of both)."""
    n_dev, w_dev = accuracy(got, truth, allow_extra, rtol, atol)
    n_orc, w_orc = accuracy(oracle32, truth, allow_extra, rtol, atol)
    qs = (99.0, 99.9, 99.99)
    pd = normalised_error_percentiles(got, truth, allow_extra, rtol, atol, qs)
    po = normalised_error_percentiles(oracle32, truth, allow_extra, rtol, atol, qs)
    log = os.environ.get("GSV_MARGIN_LOG")
    if log:
        with open(log, "a") as f:
            f.write(f"{name}\t{np.size(truth)}\tdev {n_dev}\torc {n_orc}\t"
                    f"{w_dev:.4g}\t{w_orc:.4g}\tpct dev {' '.join(f'{v:.3g}' for v in pd)}"
                    f"\torc {' '.join(f'{v:.3g}' for v in po)}\n")
    cr, ca, pf, wf = ((STRICT["count_rel"], STRICT["count_abs"], STRICT["p999"], STRICT["worst"])
                      if strict else (COUNT_SLACK_REL, COUNT_SLACK_ABS, P999_FACTOR, WORST_FACTOR))
    n_max = int(cr * n_orc + ca)
    p_max = max(0.1, pf * float(po[1]))
    w_max = max(1.0, wf * w_orc)
    assert n_dev <= n_max and float(pd[1]) <= p_max and w_dev <= w_max, (
        f"{name}: device {n_dev} elements outside rel {rtol} / abs {atol} of the binary64 "
        f"truth (99.9th percentile {float(pd[1]):.4g}, worst {w_dev:.4g} of the bound), "
        f"binary32 oracle {n_orc} ({float(po[1]):.4g}, {w_orc:.4g}); allowed {n_max} "
        f"({p_max:.4g}, {w_max:.4g})")
    return n_dev, n_orc, w_dev, w_orc


class AccuracyChecks:
    """Runs several assert_no_less_accurate comparisons and raises once, after
    all of them, listing every one that failed (so one run logs them all)."""

    def __init__(self):
        self.failures = []

    def check(self, *args, **kw):
        try:
            return assert_no_less_accurate(*args, **kw)
        except AssertionError as e:
            self.failures.append(str(e))
            return None

    def done(self):
        assert not self.failures, "\n".join(self.failures)


def l1_vol_grad(vol, target):
    """Gradient of mean |vol - target| w.r.t. vol (torch.nn.functional.l1_loss)."""
    return (np.sign(vol.astype(np.float64) - target.astype(np.float64)) / vol.size).astype(np.float32)
