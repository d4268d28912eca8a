"""Pins the oracle's voxelization (forward + backward) without the reference.

Forward: a dense fp64 evaluation written as a scatter over (tile, Gaussian)
pairs with torch — a different algorithm from the oracle's per-voxel gather —
plus closed forms of a single Gaussian and additivity over Gaussians.
Backward: torch autograd through that fp64 evaluation gives the exact
derivatives of the gated forward (voxelize.cu:368-574 computes these
analytically); the oracle must match them.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from helpers import report_close


def dense_fp64(vol, ids, bins, pr, cn, inten):
    """Scatter every (tile, Gaussian) pair's 8^3 voxels in fp64.  Returns the
    volume (D,H,W,C) as a function of leaf tensors mu (N,3), conic (N,6), I (N,C)."""
    D, H, W = vol
    Tx, Ty, Tz = O.tile_grid(vol)
    mu = torch.tensor(pr[:, :3], dtype=torch.float64, requires_grad=True)
    con = torch.tensor(cn, dtype=torch.float64, requires_grad=True)
    I = torch.tensor(inten, dtype=torch.float64, requires_grad=True)
    C = I.shape[1]
    tiles = np.repeat(np.arange(Tx * Ty * Tz), bins[:, 1] - bins[:, 0])
    g = torch.from_numpy(ids.astype(np.int64))
    t = torch.from_numpy(tiles)
    loc = torch.stack(torch.meshgrid(torch.arange(8), torch.arange(8), torch.arange(8),
                                     indexing="ij"), -1).reshape(512, 3)  # (lz, ly, lx)
    z = (t // (Tx * Ty))[:, None] * 8 + loc[None, :, 0]
    y = ((t // Tx) % Ty)[:, None] * 8 + loc[None, :, 1]
    x = (t % Tx)[:, None] * 8 + loc[None, :, 2]
    inside = (x < W) & (y < H) & (z < D)
    d = mu[g][:, None, :] - torch.stack([x, y, z], -1).double() - 0.5
    a, b, c, dd, e, f = (con[g][:, k, None] for k in range(6))
    sig = -0.5 * (a * d[..., 0] ** 2 + dd * d[..., 1] ** 2 + f * d[..., 2] ** 2) - (
        b * d[..., 0] * d[..., 1] + c * d[..., 0] * d[..., 2] + e * d[..., 1] * d[..., 2])
    alpha = torch.exp(sig)
    mean = I[g].mean(1, keepdim=True)
    keep = inside & (sig <= 0) & torch.isfinite(sig) & (alpha * mean >= 1e-6)
    contrib = torch.where(keep[..., None], I[g][:, None, :] * alpha[..., None], 0.0)
    flat = ((z * H + y) * W + x).clamp(max=D * H * W - 1)
    out = torch.zeros(D * H * W, C, dtype=torch.float64).index_add(
        0, flat.reshape(-1), contrib.reshape(-1, C))
    return out.reshape(D, H, W, C), (mu, con, I)


def _scene(n, seed, vol=(20, 24, 17), C=1):
    rng = np.random.default_rng(seed)
    D, H, W = vol
    pos = (rng.random((n, 3)) * np.array([1.0, 1.0, 1.0])).astype(np.float32)
    vs = np.array([1.0 / W, 1.0 / H, 1.0 / D])
    scale = (np.exp(rng.uniform(np.log(0.4), np.log(3.0), (n, 3))) * vs).astype(np.float32)
    q = rng.standard_normal((n, 4))
    quat = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    inten = rng.uniform(0.01, 1.0, (n, C)).astype(np.float32)
    r = O.pipeline(pos, scale, quat, inten, vol, (1.0, 1.0, 1.0), (0.5, 0.5, 0.5))
    return r, inten


@pytest.mark.parametrize("C", [1, 2, 4])
def test_forward_matches_dense_fp64(C):
    vol = (20, 24, 17)
    r, inten = _scene(80, C, vol, C)
    got, amb = O.voxelize_fwd(vol, r["gaussian_ids_sorted"], r["tile_bins"], r["pos3d_radii"],
                              r["conics"], inten, with_amb=True)
    ref, _ = dense_fp64(vol, r["gaussian_ids_sorted"], r["tile_bins"], r["pos3d_radii"],
                        r["conics"], inten)
    report_close(f"volume C={C}", got, ref.detach().numpy(), 1e-5, 1e-7, bound=amb)
    assert got.max() > 0.1


def test_forward_closed_form_single_gaussian():
    vol = (16, 16, 16)
    s = 1.3
    pr = np.array([[8.5, 8.5, 8.5, 4.0]], np.float32)  # centred on voxel (8, 8, 8)
    cn = np.array([[1 / s**2, 0, 0, 1 / s**2, 0, 1 / s**2]], np.float32)
    tmin = np.array([[0, 0, 0]], np.int32)
    tmax = np.array([[2, 2, 2]], np.int32)
    ids, bins = O.bin_and_sort(1, 8, tmin, tmax, np.array([8], np.int32), vol)
    I = np.array([[0.7]], np.float32)
    out = O.voxelize_fwd(vol, ids, bins, pr, cn, I)[..., 0]
    assert out[8, 8, 8] == pytest.approx(0.7, rel=1e-6)
    for dz, dy, dx in ((0, 0, 1), (0, 1, 0), (1, 0, 0), (1, 1, 1), (0, 3, 2)):
        r2 = dx * dx + dy * dy + dz * dz
        assert out[8 + dz, 8 + dy, 8 + dx] == pytest.approx(0.7 * math.exp(-0.5 * r2 / s**2),
                                                             rel=1e-5)
    # far voxels fall under alpha * mean < 1e-6 and are exactly zero
    far = 0.7 * np.exp(-0.5 * ((np.indices(out.shape) - 8).astype(np.float64) ** 2).sum(0) / s**2)
    assert (out[far < 0.99e-6] == 0).all()


def test_forward_additive_over_gaussians():
    vol = (24, 24, 24)
    r, inten = _scene(60, 11, vol)
    n = inten.shape[0]
    half = np.arange(n) < n // 2

    def part(mask):
        pr = np.where(mask[:, None], r["pos3d_radii"], 0).astype(np.float32)
        tmin = np.where(mask[:, None], r["tile_min"], 0).astype(np.int32)
        tmax = np.where(mask[:, None], r["tile_max"], 0).astype(np.int32)
        nt = np.where(mask, r["num_tiles_hit"], 0).astype(np.int32)
        cum = O.cumsum(nt)
        ids, bins = O.bin_and_sort(n, int(cum[-1]), tmin, tmax, cum, vol)
        return O.voxelize_fwd(vol, ids, bins, pr, r["conics"], inten)

    whole = r["volume"]
    np.testing.assert_allclose(part(half) + part(~half), whole, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("C", [1, 3])
def test_backward_matches_autograd(C):
    vol = (20, 24, 17)
    r, inten = _scene(60, 20 + C, vol, C)
    rng = np.random.default_rng(C)
    g = rng.standard_normal(vol + (C,)).astype(np.float32)
    (dp, dc, di), absum, amb = O.voxelize_bwd(vol, r["gaussian_ids_sorted"], r["tile_bins"],
                                              r["pos3d_radii"], r["conics"], inten, g,
                                              diagnostics=True)
    out, (mu, con, I) = dense_fp64(vol, r["gaussian_ids_sorted"], r["tile_bins"],
                                   r["pos3d_radii"], r["conics"], inten)
    (out * torch.from_numpy(g).double()).sum().backward()
    report_close("dmu", dp[:, :3], mu.grad.numpy(), 1e-4, 1e-6,
                 bound=1e-5 * absum[0][:, :3] + amb[0][:, :3])
    assert not dp[:, 3].any()
    report_close("dconic", dc, con.grad.numpy(), 1e-4, 1e-6, bound=1e-5 * absum[1] + amb[1])
    report_close("dintens", di, I.grad.numpy(), 1e-4, 1e-6, bound=1e-5 * absum[2] + amb[2])


def test_backward_central_difference_of_oracle_forward():
    """The oracle's own forward, differenced in the intensities (volume is
    linear in I away from the gates): sum_v g_v * vol_v(I + h e_k) changes at
    the rate dL/dI_k the backward reports."""
    vol = (16, 16, 16)
    r, inten = _scene(20, 31, vol)
    g = np.random.default_rng(4).standard_normal(vol + (1,)).astype(np.float32)
    _, _, di = O.voxelize_bwd(vol, r["gaussian_ids_sorted"], r["tile_bins"], r["pos3d_radii"],
                              r["conics"], inten, g)
    for k in (0, 5, 13):
        h = 1e-2 * inten[k, 0]
        Lp, Lm = [], []
        for sgn, acc in ((1, Lp), (-1, Lm)):
            I2 = inten.copy()
            I2[k, 0] += sgn * h
            v = O.voxelize_fwd(vol, r["gaussian_ids_sorted"], r["tile_bins"], r["pos3d_radii"],
                               r["conics"], I2)
            acc.append((v.astype(np.float64) * g).sum())
        fd = (Lp[0] - Lm[0]) / (2 * h)
        assert fd == pytest.approx(float(di[k, 0]), rel=2e-3, abs=1e-4)
