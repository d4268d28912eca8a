"""Pins the oracle's binary64 build (liboracle64.so, the truth the GPU parity
tests measure binary32 results against) without the reference.

It is the same source as the binary32 oracle with the arithmetic type
switched, so what needs pinning is that every operation really runs in
binary64 (a binary32 call or constant left in would cost ~1e-7 relative):
the checks below hold it to independent fp64 restatements at tolerances a
binary32 evaluation cannot meet (1e-9 and tighter, where the binary32 build is
held to 1e-4 to 1e-6):

- projection forward: scipy's rotation and numpy.linalg.inv (conics, centres);
- projection backward: fp64 central differences of the unnormalised-rotation
  forward (all four dquat components, dscale) and the closed form of the 1e-7
  det^2 regulariser with the reference's binary32 constant;
- voxelize forward and backward: the dense fp64 torch scatter and its autograd;
- and the binary32 build agrees with it to binary32 rounding on a
  well-conditioned scene (the two builds compute the same formulas).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import report_close
from test_oracle_projection import (_random, _well_conditioned, fp64_project,
                                    fp64_project_quadratic)
from test_oracle_voxelize import _scene, dense_fp64

F = O.f64
REG = float(np.float32(1e-7))  # the reference's binary32 constant (optim_to_render.cu:200)


def test_projection_forward_matches_scipy_fp64():
    pos, scale, quat, inten, vol, world, center = _random(2000, 17, C=2)
    pr, cn, tmin, tmax, nt = F.project_fwd(pos, scale, quat, inten, vol, world, center)
    assert pr.dtype == np.float64 and cn.dtype == np.float64
    pix, conic, _ = fp64_project(pos, scale, quat, inten, vol, world, center)
    kept = nt > 0
    assert kept.mean() > 0.9
    np.testing.assert_allclose(pr[kept, :3], pix[kept], rtol=1e-13, atol=1e-12)
    row = np.abs(conic[kept]).max(1, keepdims=True)
    report_close("binary64 conics", cn[kept], conic[kept], rtol=1e-9, atol=0.0,
                 bound=1e-10 * np.broadcast_to(row, conic[kept].shape))


def _fd(pos, scale, quat, vol, world, center, gpos, gcon, which, h):
    """Central differences of <gpos, pix> + <gcon, conic> through the
    unnormalised quadratic rotation (the function the reference differentiates)."""
    args = [a.astype(np.float64) for a in (pos, scale, quat)]
    base = args[which]
    out = np.zeros_like(base)
    for i in range(base.shape[0]):
        for k in range(base.shape[1]):
            vals = []
            for sgn in (1, -1):
                a = [x.copy() for x in args]
                a[which][i, k] += sgn * h * max(1.0, abs(base[i, k]))
                pix, conic = fp64_project_quadratic(*a, vol, world, center)
                vals.append((gpos * pix).sum() + (gcon * conic).sum())
            out[i, k] = (vals[0] - vals[1]) / (2 * h * max(1.0, abs(base[i, k])))
    return out


def test_projection_backward_matches_fp64_differences():
    """dscale and all four dquat components at rtol 1e-7 on well-conditioned
    Gaussians (det^2 >= 130: the regulariser moves ~1e-9); dpos is dpix times
    the voxel size (the reference's convention) to the last bits."""
    n = 12
    pos, scale, quat, inten, vol, world, center = _well_conditioned(n, 41)
    pr, cn, tmin, tmax, nt = F.project_fwd(pos, scale, quat, inten, vol, world, center)
    assert (nt > 0).all()
    rng = np.random.default_rng(9)
    gpos = rng.standard_normal((n, 3))
    gcon = rng.standard_normal((n, 6))
    dp, ds, dq = F.project_bwd(pos, scale, quat, vol, world, center, np.c_[gpos, np.zeros(n)],
                               gcon, pr)
    fd_s = _fd(pos, scale, quat, vol, world, center, gpos, gcon, 1, h=1e-7)
    report_close("binary64 dscale", ds, fd_s, rtol=1e-6,
                 atol=1e-8 * np.abs(fd_s).max(1, keepdims=True))
    fd_q = _fd(pos, scale, quat, vol, world, center, gpos, gcon, 2, h=1e-6)
    report_close("binary64 dquat", dq, fd_q, rtol=1e-6,
                 atol=1e-8 * np.abs(fd_q).max(1, keepdims=True))
    vs = np.array([world[2] / vol[2], world[1] / vol[1], world[0] / vol[0]])
    np.testing.assert_allclose(dp, gpos * vs, rtol=1e-15)


@pytest.mark.parametrize("s_vox", [0.2, 0.5])
def test_det_regulariser_closed_form_binary64(s_vox):
    vol, world, center = (40, 56, 48), (1.0, 1.5, 0.8), (0.5, 0.7, 0.5)
    vs = np.array([world[2] / vol[2], world[1] / vol[1], world[0] / vol[0]])
    pix = np.array([[19.3, 21.7, 13.4], [27.6, 9.2, 30.1], [5.3, 37.8, 22.9]])
    lo = np.array([center[2] - world[2] / 2, center[1] - world[1] / 2, center[0] - world[0] / 2])
    pos = (lo + pix * vs).astype(np.float32)
    scale = np.tile((s_vox * vs).astype(np.float32), (3, 1))
    quat = np.tile(np.array([1, 0, 0, 0], np.float32), (3, 1))
    inten = np.full((3, 1), 0.5, np.float32)
    pr, *_ = F.project_fwd(pos, scale, quat, inten, vol, world, center)
    gcon = np.zeros((3, 6))
    gcon[0, 0], gcon[1, 3], gcon[2, 5] = 1.5, -0.7, 2.0
    _, ds, _ = F.project_bwd(pos, scale, quat, vol, world, center, np.zeros((3, 4)), gcon, pr)
    # cov_vox = diag(s_x^2, s_y^2, s_z^2) with s_j = scale_j / vs_j (the binary32
    # scales make the three differ in their last bits, which shows at 1e-9): a
    # gradient g on conic_kk gives dL/dcov_kk = -g prod_{j != k} s_j^4 /
    # (prod_j s_j^4 + 1e-7f) and dscale_k = that * 2 s_k / vs_k (the isotropic
    # case is the binary32 test's -2 s^9 g / ((s^12 + 1e-7) vs_k))
    s_eff = scale.astype(np.float64) / vs
    want = np.zeros((3, 3))
    for r, (k, g) in enumerate(((0, 1.5), (1, -0.7), (2, 2.0))):
        s4 = s_eff[r] ** 4
        others = np.prod(np.delete(s4, k))
        want[r, k] = -2.0 * g * others * s_eff[r, k] / (vs[k] * (np.prod(s4) + REG))
    report_close(f"binary64 dscale closed form s={s_vox}", ds, want, rtol=1e-9,
                 atol=1e-12 * np.abs(want).max())


@pytest.mark.parametrize("C", [1, 3])
def test_voxelize_forward_matches_dense_fp64(C):
    vol = (20, 24, 17)
    r, inten = _scene(80, 50 + C, vol, C)
    got, amb = F.voxelize_fwd(vol, r["gaussian_ids_sorted"], r["tile_bins"], r["pos3d_radii"],
                              r["conics"], inten, with_amb=True)
    assert got.dtype == np.float64
    ref, _ = dense_fp64(vol, r["gaussian_ids_sorted"], r["tile_bins"], r["pos3d_radii"],
                        r["conics"], inten)
    report_close(f"binary64 volume C={C}", got, ref.detach().numpy(), 1e-12, 1e-16, bound=amb)
    assert got.max() > 0.1


@pytest.mark.parametrize("C", [1, 2])
def test_voxelize_backward_matches_autograd_fp64(C):
    vol = (20, 24, 17)
    r, inten = _scene(60, 60 + C, vol, C)
    g = np.random.default_rng(C + 3).standard_normal(vol + (C,))
    (dp, dc, di), absum, amb = F.voxelize_bwd(vol, r["gaussian_ids_sorted"], r["tile_bins"],
                                              r["pos3d_radii"], r["conics"], inten, g,
                                              diagnostics=True)
    out, (mu, con, I) = dense_fp64(vol, r["gaussian_ids_sorted"], r["tile_bins"],
                                   r["pos3d_radii"], r["conics"], inten)
    (out * torch.from_numpy(g)).sum().backward()
    # summation-order rounding of binary64 sums: 1e-12 x their absolute sums
    report_close("binary64 dmu", dp[:, :3], mu.grad.numpy(), 1e-10, 1e-14,
                 bound=1e-12 * absum[0][:, :3] + amb[0][:, :3])
    assert not dp[:, 3].any()
    report_close("binary64 dconic", dc, con.grad.numpy(), 1e-10, 1e-14,
                 bound=1e-12 * absum[1] + amb[1])
    report_close("binary64 dintens", di, I.grad.numpy(), 1e-10, 1e-14,
                 bound=1e-12 * absum[2] + amb[2])


def test_binary32_build_agrees_to_its_rounding():
    """The two builds evaluate the same formulas: on a well-conditioned scene
    (binary32 inputs) the binary32 chain lies within binary32 rounding of the
    binary64 one."""
    vol = (24, 24, 24)
    r32, inten = _scene(100, 71, vol, 1)
    args = (vol, r32["gaussian_ids_sorted"], r32["tile_bins"], r32["pos3d_radii"],
            r32["conics"], inten)
    v32, amb = O.voxelize_fwd(*args, with_amb=True)
    v64 = F.voxelize_fwd(*args)
    report_close("binary32 vs binary64 volume", v32, v64, 1e-5, 1e-7, bound=amb)
    g = np.random.default_rng(2).standard_normal(vol + (1,)).astype(np.float32)
    b32 = O.voxelize_bwd(*args, g)
    (b64, absum, amb) = F.voxelize_bwd(*args, g, diagnostics=True)
    for nm, a, b, s, m in zip(("dpos3d_radii", "dconics", "dintensities"), b32, b64, absum, amb):
        report_close(f"binary32 vs binary64 {nm}", a, b, 1e-4, 1e-6, bound=2e-5 * s + m)
