"""Pins the oracle's projection (forward + backward) without the reference.

Forward: an independent fp64 restatement built from textbook pieces —
scipy's quaternion->rotation, Sigma = R S^2 R^T, per-axis voxel scaling and
numpy.linalg.inv — must agree with the oracle's binary32 GLM-order arithmetic;
integer tile boxes must agree exactly wherever fp64 is not within rounding of a
tile boundary.  Closed forms and hand-computed boxes catch axis / transpose
mistakes that a random test could average away.

Backward: fp64 central finite differences of that independent forward give the
true derivatives; the reference's backward (optim_to_render.cu:246-336)
matches them for scale3d, for quat on the unit sphere's tangent space (it omits
the normalisation Jacobian), and for pos3d up to its documented factor: it
returns dpix * voxel_size where the derivative is dpix / voxel_size.  Tighter
pins: all four dquat components (the radial one included) against central
differences through the quaternion's quadratic rotation polynomial without
normalisation, which is the function the reference differentiates
(optim_to_render_helpers.cuh:15-75); dscale at rtol 1e-4 on well-conditioned
Gaussians; and the 1e-7 regulariser on det^2 (optim_to_render.cu:200) through
its closed form for isotropic Gaussians of 0.2-0.5 voxel.
"""
import math

import numpy as np
import pytest
from scipy.spatial.transform import Rotation

import oracle as O
from helpers import report_close


def fp64_project(pos, scale, quat, inten, vol, world, center):
    """Independent fp64 projection. Returns pix (N,3), conic6 (N,6), cov_vox (N,3,3)."""
    D, H, W = vol
    wz, wy, wx = world
    cz, cy, cx = center
    vs = np.array([wx / W, wy / H, wz / D])  # voxel size along x, y, z
    c = np.array([cx, cy, cz])
    w = np.array([wx, wy, wz])
    pix = (pos.astype(np.float64) - c + 0.5 * w) / vs
    q = quat.astype(np.float64)
    R = Rotation.from_quat(np.c_[q[:, 1:], q[:, :1]]).as_matrix()  # scipy: scalar last
    S2 = np.einsum("ni,ij->nij", scale.astype(np.float64) ** 2, np.eye(3))
    cov = R @ S2 @ np.transpose(R, (0, 2, 1))
    cov_vox = cov / (vs[:, None] * vs[None, :])
    Q = np.linalg.inv(cov_vox)
    conic = np.stack([Q[:, 0, 0], Q[:, 0, 1], Q[:, 0, 2], Q[:, 1, 1], Q[:, 1, 2], Q[:, 2, 2]], 1)
    return pix, conic, cov_vox


def fp64_boxes(pix, cov_vox, inten, vol):
    Tx, Ty, Tz = O.tile_grid(vol)
    m = inten.astype(np.float64).mean(1)
    with np.errstate(invalid="ignore", divide="ignore"):
        ext = np.sqrt(2.0 * np.log(m * 1e6))
    ext = np.where(np.isnan(ext), 3.0, np.minimum(3.0, ext))
    r3 = np.maximum(0.0, np.sqrt(np.diagonal(cov_vox, axis1=1, axis2=2)) * ext[:, None] - 0.5)
    lo_f = (pix - r3) / 8.0
    hi_f = (pix + r3 + 7.0) / 8.0
    T = np.array([Tx, Ty, Tz])
    lo = np.clip(np.trunc(lo_f), 0, T).astype(np.int64)
    hi = np.clip(np.trunc(hi_f), 0, T).astype(np.int64)
    near = lambda v: np.abs(v - np.round(v)) < 1e-4
    return lo, hi, near(lo_f) | near(hi_f)


def _random(n, seed, vol=(40, 56, 48), world=(1.0, 1.5, 0.8), center=(0.5, 0.7, 0.5), C=1):
    rng = np.random.default_rng(seed)
    wz, wy, wx = world
    cz, cy, cx = center
    lo = np.array([cx - wx / 2, cy - wy / 2, cz - wz / 2])
    pos = (lo + rng.random((n, 3)) * np.array([wx, wy, wz])).astype(np.float32)
    vs = np.array([wx / vol[2], wy / vol[1], wz / vol[0]])
    scale = (np.exp(rng.uniform(np.log(0.5), np.log(5.0), (n, 3))) * vs).astype(np.float32)
    q = rng.standard_normal((n, 4))
    quat = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    inten = rng.uniform(0.05, 1.0, (n, C)).astype(np.float32)
    return pos, scale, quat, inten, vol, world, center


@pytest.mark.parametrize("C", [1, 3])
def test_forward_matches_independent_fp64(C):
    pos, scale, quat, inten, vol, world, center = _random(3000, 7, C=C)
    pr, cn, tmin, tmax, nt = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    pix, conic, cov_vox = fp64_project(pos, scale, quat, inten, vol, world, center)
    kept = nt > 0
    assert kept.mean() > 0.9
    np.testing.assert_allclose(pr[kept, :3], pix[kept], rtol=1e-6, atol=1e-4)
    scale_c = np.abs(conic[kept]).max(1, keepdims=True)
    report_close("conics", cn[kept], conic[kept], rtol=2e-3, atol=0.0,
                 bound=2e-4 * np.broadcast_to(scale_c, conic[kept].shape))
    lo, hi, ambiguous = fp64_boxes(pix, cov_vox, inten, vol)
    ok = kept[:, None] & ~ambiguous
    assert ok.mean() > 0.85
    np.testing.assert_array_equal(tmin[ok], lo[ok])
    np.testing.assert_array_equal(tmax[ok], hi[ok])
    np.testing.assert_array_equal(nt, np.where(kept, np.prod(tmax - tmin, 1), 0))


def test_closed_form_identity_isotropic():
    vol, world, center = (64, 64, 64), (1.0, 1.0, 1.0), (0.5, 0.5, 0.5)
    s_vox = 2.0
    pos = np.array([[0.5, 0.5, 0.5]], np.float32)
    scale = np.full((1, 3), s_vox / 64, np.float32)
    quat = np.array([[1, 0, 0, 0]], np.float32)
    inten = np.array([[0.5]], np.float32)
    pr, cn, tmin, tmax, nt = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    # pix = 32; conic = diag(1/4); radius = ceil(3*2) = 6; r3 = 2*3-0.5 = 5.5
    np.testing.assert_allclose(pr[0], [32, 32, 32, 6], rtol=1e-6)
    np.testing.assert_allclose(cn[0], [0.25, 0, 0, 0.25, 0, 0.25], rtol=1e-5, atol=1e-7)
    # tile_min = trunc((32-5.5)/8) = 3, tile_max = trunc((32+5.5+7)/8) = 5
    np.testing.assert_array_equal(tmin[0], [3, 3, 3])
    np.testing.assert_array_equal(tmax[0], [5, 5, 5])
    assert nt[0] == 8


def test_axes_follow_zyx_tuples_and_xyz_positions():
    """A Gaussian stretched along x in a non-cubic, off-centre volume: its box is
    wide along x (the W axis), and the voxel sizes come from the matching world
    extents; a 90-degree turn about z swaps the x and y widths."""
    vol, world, center = (32, 48, 80), (0.5, 1.5, 2.0), (1.0, 0.0, -1.0)
    vs = np.array([2.0 / 80, 1.5 / 48, 0.5 / 32])  # x, y, z voxel sizes
    pos = np.array([[-1.0, 0.0, 1.0]], np.float32)  # volume centre (x, y, z)
    scale = (np.array([[6.0, 1.0, 1.0]]) * vs).astype(np.float32)
    inten = np.ones((1, 1), np.float32)
    q0 = np.array([[1, 0, 0, 0]], np.float32)
    qz = np.array([[math.cos(math.pi / 4), 0, 0, math.sin(math.pi / 4)]], np.float32)
    pr, cn, tmin, tmax, _ = O.project_fwd(pos, scale, q0, inten, vol, world, center)
    np.testing.assert_allclose(pr[0, :3], [40, 24, 16], atol=1e-4)
    wid = tmax[0] - tmin[0]
    assert wid[0] > wid[1] and wid[0] > wid[2]
    np.testing.assert_allclose(cn[0, [0, 3, 5]], [1 / 36, 1.0, 1.0], rtol=1e-4)
    pr2, cn2, tmin2, tmax2, _ = O.project_fwd(pos, scale, qz, inten, vol, world, center)
    # after the turn the long axis is y: the y variance is (6 vs_x / vs_y)^2
    np.testing.assert_allclose(1 / cn2[0, 3], (6 * vs[0] / vs[1]) ** 2, rtol=1e-4)
    wid2 = tmax2[0] - tmin2[0]
    assert wid2[1] > wid2[0]


def test_special_rows():
    vol, world, center = (32, 32, 32), (1.0, 1.0, 1.0), (0.5, 0.5, 0.5)
    pos = np.full((6, 3), 0.5, np.float32)      # pix = 16
    scale = np.full((6, 3), 4.0 / 32, np.float32)  # 4 voxels
    quat = np.tile(np.array([1, 0, 0, 0], np.float32), (6, 1))
    inten = np.array([[0.5], [0.0], [-1.0], [2e-6], [0.5], [0.5]], np.float32)
    scale[4] = [0.0, 0.1, 0.1]          # det == 0 -> culled
    pos[5] = [3.0, 0.5, 0.5]            # outside by more than the radius -> culled
    pr, cn, tmin, tmax, nt = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    for r in (4, 5):
        assert not pr[r].any() and not cn[r].any() and not tmin[r].any() and not tmax[r].any()
        assert nt[r] == 0
    # extent: log(0) = -inf and log(<0) = NaN both give fminf(3, NaN) = 3
    np.testing.assert_array_equal(tmin[1], tmin[0])
    np.testing.assert_array_equal(tmin[2], tmin[0])
    # extent 3: r3 = 11.5 -> tiles [0, 4) per axis
    np.testing.assert_array_equal(tmin[0], [0, 0, 0])
    np.testing.assert_array_equal(tmax[0], [4, 4, 4])
    # mean*1e6 = 2 -> extent = sqrt(2 ln 2) ~ 1.177, r3 ~ 4.21 -> tiles [1, 3)
    np.testing.assert_array_equal(tmin[3], [1, 1, 1])
    np.testing.assert_array_equal(tmax[3], [3, 3, 3])
    assert nt[0] == 64 and nt[3] == 8


def _loss_fd(pos, scale, quat, inten, vol, world, center, gpos, gcon, which, h=1e-6):
    """Central differences of L = <gpos, pix> + <gcon, conic> in fp64."""
    args = [pos.astype(np.float64), scale.astype(np.float64), quat.astype(np.float64)]
    base = args[which]
    grad = np.zeros_like(base)
    for i in range(base.shape[0]):
        for k in range(base.shape[1]):
            vals = []
            for sgn in (1, -1):
                a = [x.copy() for x in args]
                a[which][i, k] += sgn * h
                if which == 2:
                    a[2][i] /= np.linalg.norm(a[2][i])  # the forward normalises
                pix, conic, _ = fp64_project(a[0], a[1], a[2], inten, vol, world, center)
                vals.append((gpos * pix).sum() + (gcon * conic).sum())
            grad[i, k] = (vals[0] - vals[1]) / (2 * h)
    return grad


def test_backward_matches_finite_differences():
    pos, scale, quat, inten, vol, world, center = _random(12, 3)
    pr, cn, tmin, tmax, nt = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    assert (nt > 0).all()
    rng = np.random.default_rng(1)
    gpos = rng.standard_normal((12, 3))
    gcon = rng.standard_normal((12, 6))
    dpr = np.c_[gpos, np.zeros(12)].astype(np.float32)
    dp, ds, dq = O.project_bwd(pos, scale, quat, vol, world, center, dpr, gcon.astype(np.float32), pr)
    fd_scale = _loss_fd(pos, scale, quat, inten, vol, world, center, gpos, gcon, 1, h=1e-7)
    np.testing.assert_allclose(ds, fd_scale, rtol=2e-3, atol=1e-3 * np.abs(fd_scale).max())
    fd_quat = _loss_fd(pos, scale, quat, inten, vol, world, center, gpos, gcon, 2, h=1e-6)
    q = quat.astype(np.float64)
    tangential = dq - (dq * q).sum(1, keepdims=True) * q
    np.testing.assert_allclose(tangential, fd_quat, rtol=2e-3, atol=1e-3 * np.abs(fd_quat).max())
    # dpos = dpix * voxel_size (the reference's convention); true derivative = dpix / voxel_size
    vs = np.array([world[2] / vol[2], world[1] / vol[1], world[0] / vol[0]])
    np.testing.assert_allclose(dp, gpos * vs, rtol=1e-6)
    fd_pos = _loss_fd(pos, scale, quat, inten, vol, world, center, gpos, gcon, 0, h=1e-6)
    np.testing.assert_allclose(dp, fd_pos * vs ** 2, rtol=1e-4, atol=1e-6)


def test_backward_skips_culled_rows():
    pos, scale, quat, inten, vol, world, center = _random(4, 5)
    pr, *_ = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    pr = pr.copy()
    pr[1, 3] = 0.0
    g = np.ones((4, 6), np.float32)
    dp, ds, dq = O.project_bwd(pos, scale, quat, vol, world, center, np.ones((4, 4), np.float32), g, pr)
    assert not dp[1].any() and not ds[1].any() and not dq[1].any()
    assert dp[0].any() and ds[0].any()


def fp64_project_quadratic(pos, scale, quat, vol, world, center):
    """fp64 projection whose rotation is the quadratic polynomial R(q) of a
    quaternion [w, x, y, z] with no normalisation (the entries 1 - 2(y^2 + z^2),
    2(xy - wz), ... of the unit-quaternion rotation matrix, evaluated at q as
    given).  At unit q it is the rotation of scipy's restatement above; its
    derivative with respect to all four components is what a backward without
    the normalisation Jacobian returns (optim_to_render_helpers.cuh:51-75
    differentiates these entries; :15-36 builds them)."""
    D, H, W = vol
    wz, wy, wx = world
    cz, cy, cx = center
    vs = np.array([wx / W, wy / H, wz / D])
    pix = (pos - np.array([cx, cy, cz]) + 0.5 * np.array([wx, wy, wz])) / vs
    w, x, y, z = (quat[:, i] for i in range(4))
    R = np.stack([
        np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        np.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        np.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], 1)
    S2 = np.einsum("ni,ij->nij", scale ** 2, np.eye(3))
    cov_vox = (R @ S2 @ np.transpose(R, (0, 2, 1))) / (vs[:, None] * vs[None, :])
    Q = np.linalg.inv(cov_vox)
    conic = np.stack([Q[:, 0, 0], Q[:, 0, 1], Q[:, 0, 2], Q[:, 1, 1], Q[:, 1, 2], Q[:, 2, 2]], 1)
    return pix, conic


def _well_conditioned(n, seed):
    """Random Gaussians of 1.5-5 voxels per axis: det(cov_vox)^2 >= 1.5^12 ~ 130,
    so the backward's 1e-7 regulariser on det^2 moves nothing above ~1e-9."""
    pos, scale, quat, inten, vol, world, center = _random(n, seed)
    vs = np.array([world[2] / vol[2], world[1] / vol[1], world[0] / vol[0]])
    rng = np.random.default_rng(seed + 100)
    scale = (np.exp(rng.uniform(np.log(1.5), np.log(5.0), (n, 3))) * vs).astype(np.float32)
    return pos, scale, quat, inten, vol, world, center


def test_dquat_all_four_components_match_unnormalised_rotation():
    """All four dquat components, the radial one included, against fp64 central
    differences through R(q) without normalisation, at unit q.  A backward that
    applied the normalisation Jacobian (the tangential projection) would lose
    the radial part and fail here."""
    pos, scale, quat, inten, vol, world, center = _well_conditioned(16, 21)
    pr, cn, tmin, tmax, nt = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    assert (nt > 0).all()
    rng = np.random.default_rng(5)
    gpos = rng.standard_normal((16, 3))
    gcon = rng.standard_normal((16, 6))
    dpr = np.c_[gpos, np.zeros(16)].astype(np.float32)
    _, _, dq = O.project_bwd(pos, scale, quat, vol, world, center, dpr,
                             gcon.astype(np.float32), pr)
    p64, s64, q64 = (a.astype(np.float64) for a in (pos, scale, quat))
    h = 1e-6
    fd = np.zeros((16, 4))
    for i in range(16):
        for k in range(4):
            vals = []
            for sgn in (1, -1):
                q = q64.copy()
                q[i, k] += sgn * h
                pix, conic = fp64_project_quadratic(p64, s64, q, vol, world, center)
                vals.append((gpos * pix).sum() + (gcon * conic).sum())
            fd[i, k] = (vals[0] - vals[1]) / (2 * h)
    radial = np.abs((fd * q64).sum(1))
    tangential = np.abs(fd - (fd * q64).sum(1, keepdims=True) * q64).max(1)
    assert (radial > 0.05 * tangential).sum() >= 8, "scene must exercise the radial part"
    row = np.abs(fd).max(1, keepdims=True)
    report_close("dquat (all four components)", dq, fd, rtol=1e-4, atol=1e-5 * row)


def test_dscale_matches_finite_differences_tightly():
    """dscale at rtol 1e-4 where det^2 >> 1e-7 (the regulariser is then below
    1e-9 relative)."""
    pos, scale, quat, inten, vol, world, center = _well_conditioned(16, 22)
    pr, cn, tmin, tmax, nt = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    assert (nt > 0).all()
    rng = np.random.default_rng(6)
    gpos = rng.standard_normal((16, 3))
    gcon = rng.standard_normal((16, 6))
    dpr = np.c_[gpos, np.zeros(16)].astype(np.float32)
    _, ds, _ = O.project_bwd(pos, scale, quat, vol, world, center, dpr,
                             gcon.astype(np.float32), pr)
    fd = _loss_fd(pos, scale, quat, inten, vol, world, center, gpos, gcon, 1, h=1e-8)
    row = np.abs(fd).max(1, keepdims=True)
    report_close("dscale (well conditioned)", ds, fd, rtol=1e-4, atol=1e-5 * row)


def regularised_dscale(s_vox, vs, g):
    """Closed form of the reference's dscale for an identity-quaternion Gaussian
    that is isotropic in voxel units (cov_vox = s^2 I, det = s^6) with a
    gradient g on one diagonal conic element: the adjugate derivative scaled by
    1/(det^2 + 1e-7) (optim_to_render.cu:199-226) gives dL/dcov_kk =
    -s^8 g / (s^12 + 1e-7), and the chain through cov = (S R)^T (S R) with
    S = s vs (:300-321) gives dscale_k = -2 s^9 g / ((s^12 + 1e-7) vs_k).
    Without the regulariser it is the true derivative -2 g / (s^3 vs_k)."""
    return -2.0 * s_vox ** 9 * g / ((s_vox ** 12 + 1e-7) * vs)


@pytest.mark.parametrize("s_vox", [0.2, 0.3, 0.45, 0.5])
def test_det_regulariser_closed_form(s_vox):
    """The 1e-7 on det^2: dominant at 0.2 voxel (s^12 = 4e-9), comparable at 0.3
    (5e-7), a 1.4e-3 relative effect at 0.45 and 4e-4 at 0.5, each above the
    1e-4 tolerance.  Non-cubic voxels, one conic diagonal element per row, so
    the x/y/z voxel-size mapping is pinned too."""
    vol, world, center = (40, 56, 48), (1.0, 1.5, 0.8), (0.5, 0.7, 0.5)
    vs = np.array([world[2] / vol[2], world[1] / vol[1], world[0] / vol[0]])  # x, y, z
    # three Gaussians inside the volume, off tile boundaries
    pix = np.array([[19.3, 21.7, 13.4], [27.6, 9.2, 30.1], [5.3, 37.8, 22.9]])
    lo = np.array([center[2] - world[2] / 2, center[1] - world[1] / 2, center[0] - world[0] / 2])
    pos = (lo + pix * vs).astype(np.float32)
    scale = np.tile((s_vox * vs).astype(np.float32), (3, 1))
    quat = np.tile(np.array([1, 0, 0, 0], np.float32), (3, 1))
    inten = np.full((3, 1), 0.5, np.float32)
    pr, cn, tmin, tmax, nt = O.project_fwd(pos, scale, quat, inten, vol, world, center)
    assert (pr[:, 3] > 0).all()
    gcon = np.zeros((3, 6), np.float32)
    gcon[0, 0], gcon[1, 3], gcon[2, 5] = 1.5, -0.7, 2.0   # xx, yy, zz
    _, ds, dq = O.project_bwd(pos, scale, quat, vol, world, center,
                              np.zeros((3, 4), np.float32), gcon, pr)
    # the closed form uses the binary32 scale's own voxel extent
    s_eff = scale.astype(np.float64) / vs
    want = np.zeros((3, 3))
    for r, (k, g) in enumerate(((0, 1.5), (1, -0.7), (2, 2.0))):
        want[r, k] = regularised_dscale(s_eff[r, k], vs[k], g)
    report_close(f"dscale closed form s={s_vox}", ds, want, rtol=1e-4,
                 atol=1e-6 * np.abs(want).max())
    unregularised = -2.0 * np.array([1.5, -0.7, 2.0]) / (s_eff[0] ** 3 * vs)
    gap = np.abs(np.diag(want) - unregularised) / np.abs(unregularised)
    assert (gap > 1e-4).all(), "the regulariser must be visible at this size"
    assert np.abs(dq).max() <= 1e-6 * np.abs(want).max()
