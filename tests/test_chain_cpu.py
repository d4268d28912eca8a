"""The chained row evaluation of the voxelize kernels, checked on the CPU.

Both voxelize kernels form most exp2 values of an 8-voxel row as products
(an anchor 2^E and a step along the row, times per-Gaussian column factors:
2^(A2 uc^2 - K) about the tile centre in the forward, 2^(A2 dx_u^2 - K) about
the Gaussian's centre in the backward) and rely on binary32 flush-to-zero for
the reference's 1e-6 gate: a product below 2^-126 is 0.  That is only the gate if no factor of a chain flushes before a
passing voxel and nothing overflows, which the choice of K guarantees for the
pairs that qualify (csrc/voxelize.hip: the forward's record set-up and
chain_shift).  This test restates those rules in numpy (binary32 with
flush-to-zero emulated after every product) and compares every voxel of every
row of qualifying (tile, Gaussian) pairs with exp2 of the exactly computed
exponent: the gate decisions must agree except within 1e-4 (log2 units) of the
threshold, and the values within 5e-5 relative.  Scenes: cfg1's rotated
anisotropic Gaussians, narrow ones (0.15-0.6 voxel, steep rows), and cfg5's
mixture.
"""
import numpy as np
import pytest

import oracle as O
from gs_voxelizer import synthetic as S
from helpers import small_config

L2E = 1.4426950408889634
F32 = np.float32
TINY = F32(2.0 ** -126)


def _ftz(x):
    x = np.asarray(x, np.float32)
    return np.where(np.abs(x) < TINY, F32(0), x).astype(np.float32)


def _exp2(x):
    with np.errstate(over="ignore"):
        return _ftz(np.exp2(np.asarray(x, np.float32)))


def _mul(a, b):
    # inf * 0 arises only for pairs that do not qualify (checked finite below)
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        return _ftz(np.asarray(a, np.float32) * np.asarray(b, np.float32))


def _pairs(work, max_pairs, seed):
    """Per (tile, Gaussian) pair of a sample: the conic, the gate offset and the
    Gaussian centre relative to the tile centre (voxel units)."""
    cfg = work.cfg
    pr, cn, tmin, tmax, _ = O.project_fwd(work.pos3d.numpy(), work.scale3d.numpy(),
                                          work.quat.numpy(), work.intensities.numpy(), cfg.vol,
                                          cfg.world, cfg.center)
    inten = work.intensities.numpy().reshape(pr.shape[0], -1)
    rows = []
    for g in np.random.default_rng(seed).permutation(pr.shape[0]):
        (x0, y0, z0), (x1, y1, z1) = tmin[g], tmax[g]
        mean = float(inten[g].mean())
        if x1 <= x0 or y1 <= y0 or z1 <= z0 or not mean > 0:
            continue
        t2 = float(F32(np.log2(1e-6) - np.log2(F32(mean))))
        if t2 > 0 or t2 < -60:
            continue
        for tz in range(z0, z1):
            for ty in range(y0, y1):
                for tx in range(x0, x1):
                    c = pr[g, :3].astype(np.float32) - np.float32([tx * 8, ty * 8, tz * 8]) - F32(4)
                    rows.append(np.concatenate([c, cn[g], [t2]]))
        if len(rows) >= max_pairs:
            break
    return np.asarray(rows[:max_pairs], np.float64)


def _grid():
    uc = np.arange(8) - 3.5                      # x offset of voxel u from the tile centre
    ly = np.arange(64) & 7
    lz = np.arange(64) >> 3
    return uc, ly - 3.5, lz - 3.5                # row offsets (py, pz) of lane = row


def _exact_exponent(P):
    """sigma2 + off in binary64 for every pair, row and voxel: (N, 64, 8)."""
    uc, py, pz = _grid()
    cx, cy, cz = (P[:, i][:, None, None] for i in range(3))
    a, b, c, d, e, f = (P[:, 3 + i][:, None, None] for i in range(6))
    t2 = P[:, 9][:, None, None]
    dx = cx - uc[None, None, :]
    dy = cy - py[None, :, None]
    dz = cz - pz[None, :, None]
    q = a * dx * dx + 2 * b * dx * dy + 2 * c * dx * dz + d * dy * dy + 2 * e * dy * dz + f * dz * dz
    return -0.5 * L2E * q - (t2 + 126.0)


def _check(name, s_exact, got, mask):
    """Gate decisions and values of the chained rows against exp2 of the exact
    exponent, for the pairs in mask."""
    s = s_exact[mask]
    ref = _exp2(s.astype(np.float32))
    g = got[mask]
    assert np.isfinite(g).all(), f"{name}: a qualifying pair overflowed"
    amb = np.abs(s + 126.0) < 1e-4
    mismatch = ((g > 0) != (ref > 0)) & ~amb
    assert not mismatch.any(), f"{name}: {int(mismatch.sum())} gate decisions differ"
    both = (g > 0) & (ref > 0)
    rel = np.abs(g[both].astype(np.float64) / ref[both] - 1.0)
    assert rel.size == 0 or rel.max() <= 5e-5, f"{name}: max relative difference {rel.max():.3g}"
    return int(mask.sum()), int(both.sum())


def _forward_chains(P):
    """The forward's rows (lane = row (py, pz)), as k_vox_fwd forms them."""
    uc, py, pz = _grid()
    cx, cy, cz = (P[:, i].astype(np.float32) for i in range(3))
    a, b, c, d, e, f = (P[:, 3 + i].astype(np.float32) for i in range(6))
    t2 = P[:, 9].astype(np.float32)
    off = -(t2.astype(np.float64) + 126.0)
    A2 = (F32(-0.5 * L2E) * a).astype(np.float64)
    bb, cc = (F32(-L2E) * b).astype(np.float64), (F32(-L2E) * c).astype(np.float64)
    dd, ee = (F32(-0.5 * L2E) * d).astype(np.float64), (F32(-L2E) * e).astype(np.float64)
    ff = (F32(-0.5 * L2E) * f).astype(np.float64)
    X, Y, Z = (v.astype(np.float64) for v in (cx, cy, cz))
    t1 = 2.0 * A2 * X + bb * Y + cc * Z
    rec0, rec1, rec2 = t1.astype(np.float32), (-bb).astype(np.float32), (-cc).astype(np.float32)
    t0 = X * (A2 * X + bb * Y + cc * Z) + Y * (dd * Y + ee * Z) + ff * Z * Z
    ty = -(bb * X + 2.0 * dd * Y + ee * Z)
    tz = -(cc * X + ee * Y + 2.0 * ff * Z)
    bound_t1 = (np.abs(rec0) + F32(3.5) * (np.abs(rec1) + np.abs(rec2))) * F32(1.001)
    K = np.floor(F32(120.0) - F32(12.25) * np.abs(A2.astype(np.float32)))
    one_way = np.ceil(F32(7.0) * bound_t1) + 2 <= K
    chain = one_way | (np.ceil(F32(4.0) * bound_t1) + 2 <= K)
    at = np.where(one_way, -3.5, 0.5)
    rec3 = (t0 - at * t1 + off + K).astype(np.float32)
    rec4 = (ty - at * rec1.astype(np.float64)).astype(np.float32)
    rec5 = (tz - at * rec2.astype(np.float64)).astype(np.float32)
    k = np.arange(4) + 0.5
    with np.errstate(over="ignore"):  # K < 0 only for pairs that do not qualify
        G = _ftz(np.ldexp(_exp2(A2.astype(np.float32)[:, None] * (k * k).astype(np.float32)),
                          -K.astype(np.int64)[:, None]))                   # (N, 4)
    pyv, pzv = py[None, :], pz[None, :]
    T1 = (rec0[:, None] + rec1[:, None] * pyv + rec2[:, None] * pzv).astype(np.float32)
    E0 = (rec3[:, None] + rec4[:, None] * pyv + rec5[:, None] * pzv
          + dd[:, None] * pyv * pyv + ee[:, None] * pyv * pzv + ff[:, None] * pzv * pzv
          ).astype(np.float32)                                               # (N, 64)
    out = np.zeros(E0.shape + (8,), np.float32)
    idx = [3, 2, 1, 0, 0, 1, 2, 3]                                          # |uc| - 0.5 per u
    # one-way: from uc = -3.5, step 2^-T1
    step = _exp2(-T1)
    ev = _exp2(E0)
    ow = np.zeros_like(out)
    for u in range(8):
        ow[..., u] = _mul(ev, G[:, idx[u]][:, None])
        ev = _mul(ev, step)
    # centre-out: anchor at uc = +0.5, steps both ways, uc = -0.5 one step left
    step_r, step_l = _exp2(-T1), _exp2(T1)
    er = _exp2(E0)
    el = _mul(er, step_l)
    co = np.zeros_like(out)
    for kk in range(4):
        co[..., 4 + kk] = _mul(er, G[:, kk][:, None])
        co[..., 3 - kk] = _mul(el, G[:, kk][:, None])
        er, el = _mul(er, step_r), _mul(el, step_l)
    out = np.where(one_way[:, None, None], ow, co)
    return out, chain


def _f(x):
    return np.asarray(x, np.float64).astype(np.float32)


def _fma(a, b, c):
    """fmaf in binary32 with flush-to-zero (the product and sum in binary64,
    rounded once: exact for the magnitudes here)."""
    with np.errstate(over="ignore", invalid="ignore"):
        return _ftz(np.float64(a) * np.float64(b) + np.float64(c))


def _backward_chains(P):
    """The backward's rows (lane = pair, rows walked in order), as pair_moments
    with kChain forms them: a_u = 2^E_u * G_u with the column factors
    G_u = 2^(A2 (dx_u - d)^2 - K) (with the rounding residual of the
    exponent) and E_u linear in u, 2^E at u = 0 and u = 4 stepped along the
    row; and chain_shift's choice of d (0, the Gaussian's centre, or mx, the
    tile's) and K.  Returns (a, qualifies, excluded, centred): excluded are the
    pairs that pass the Gaussian-centred conditions but the dead-row bounds
    and have no tile-centred fallback, centred those that take d = 0."""
    uc, py, pz = _grid()
    F = np.float32
    mx, my, mz = (P[:, i].astype(F) for i in range(3))
    ca, cb, cc_, cd, ce, cf = (P[:, 3 + i].astype(F) for i in range(6))
    t2 = P[:, 9].astype(F)
    off = (-(t2 + F(126.0))).astype(F)
    A2 = F(-0.5 * L2E) * ca
    Bn, Cn = F(-L2E) * cb, F(-L2E) * cc_
    Dn, En, Fn = F(-0.5 * L2E) * cd, F(-L2E) * ce, F(-0.5 * L2E) * cf
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        k2 = (F(-2.0 * 0.693147180559945309) * t2).astype(F)
        i11 = (F(1) / np.sqrt(ca)).astype(F)
        l21, l31 = cb * i11, cc_ * i11
        t22 = _fma(-l21, l21, cd)
        i22 = (F(1) / np.sqrt(t22)).astype(F)
        l32 = _f(_fma(-l31, l21, ce) * i22)
        t33 = _fma(-l32, l32, _fma(-l31, l31, cf))
        y2 = Bn * i22
        y3 = _f(_fma(-l32, y2, Cn) * (F(1) / np.sqrt(t33)).astype(F))
        m_ell = np.sqrt(np.maximum(k2 * _fma(y2, y2, y3 * y3), F(0))).astype(F)
        m_ell = np.where((t22 > F(1e-3) * cd) & (t33 > F(1e-3) * cf), m_ell,
                         np.float32(np.inf)).astype(F)
        r1_tile = _f(np.abs(_fma(Bn, my, Cn * mz)) + F(3.5) * (np.abs(Bn) + np.abs(Cn)))
        # d = 0
        cfx = _fma(cd, cf, -(ce * ce))
        det = _f(ca * cfx - cb * _fma(cb, cf, -(cc_ * ce)) + cc_ * _fma(cb, ce, -(cc_ * cd)))
        dx_max = _f(np.abs(mx) + F(3.5))
        cond = ((cfx > F(1e-3) * (cd * cf)) & (det > F(1e-3) * (ca * cfx)) & (det > F(2.0 ** -100))
                & (det < F(2.0 ** 100)) & (r1_tile < F(120.0)))
        g_ell = _f(A2 * _f(k2 * cfx * _f(F(1) / det)))
        g_min = np.maximum(g_ell, _f(A2 * (dx_max * dx_max)))
        Kmax = np.floor(np.minimum(F(120.0), F(125.0) + F(1.001) * g_min)).astype(F)
        M0 = (np.minimum(r1_tile, m_ell) * F(1.001) + F(0.01)).astype(F)
        Kmin = np.ceil(F(3.0) * M0) + 2
        K0 = np.minimum(Kmax, np.maximum(Kmin, np.floor(F(126.5) + t2))).astype(F)
        live0 = cond & (Kmin <= K0)
        dead0 = np.minimum(-A2 * dx_max, r1_tile) * dx_max + K0 < F(190.0)
        centred = live0 & dead0
        # d = mx
        m_tile = _f(np.abs(_fma(F(2.0) * A2, mx, _fma(Bn, my, Cn * mz))) +
                    F(3.5) * (np.abs(Bn) + np.abs(Cn)))
        K1 = np.floor(F(120.0) - F(12.25) * np.abs(A2)).astype(F)
        m_reach = (np.abs(F(2) * A2) * (F(3.5) + np.sqrt(np.maximum(k2 / ca, F(0))))).astype(F)
        M1 = (np.minimum(m_tile, np.minimum(np.abs(F(2) * A2 * mx) + m_ell, m_reach)) * F(1.001)
              + F(0.01)).astype(F)
        tile_ok = (m_tile < F(120.0)) & (np.ceil(F(3.0) * M1) + 2 <= K1)
    qualifies = centred | tile_ok
    K = np.where(centred, K0, np.where(tile_ok, K1, np.where(live0, K0, F(2.0)))).astype(F)
    d = np.where(centred | ~tile_ok, F(0), mx).astype(F)
    dxu = _f(mx[:, None] - uc[None, :].astype(F))                      # (N, 8)
    x = np.where((d == 0)[:, None], dxu, uc[None, :].astype(F)).astype(F)
    p = _f(A2[:, None] * x)
    plo = _fma(A2[:, None], x, -p)
    hi = _f(p * x)
    lo = _fma(plo, x, _fma(p, x, -hi))
    with np.errstate(over="ignore"):
        G = _ftz(np.ldexp(np.float64(_f(np.float64(_exp2(hi)) * _fma(lo, F(0.693147180559945309), F(1)))),
                          -K.astype(np.int64)[:, None]))
    c0 = _fma(-A2 * d, d, _f(off + K))
    s0 = _f(F(2.0) * A2 * d)
    out = np.zeros((P.shape[0], 64, 8), np.float32)
    for lz in range(8):
        dz = _f(mz - F(lz - 3.5))
        Cdz, Edz = _fma(Cn, dz, s0), _f(En * dz)
        R0z = _fma(_f(Fn * dz), dz, c0)
        for ly in range(8):
            row = lz * 8 + ly
            dy = _f(my - F(ly - 3.5))
            R1 = _fma(Bn, dy, Cdz)
            R0 = _fma(_fma(Dn, dy, Edz), dy, R0z)
            step = _exp2(-R1)
            e1 = _exp2(_fma(dxu[:, 0], R1, R0))
            e2 = _exp2(_fma(dxu[:, 4], R1, R0))
            for k in range(4):
                out[:, row, k] = _mul(e1, G[:, k])
                out[:, row, 4 + k] = _mul(e2, G[:, 4 + k])
                e1, e2 = _mul(e1, step), _mul(e2, step)
    return out, qualifies, live0 & ~dead0 & ~tile_ok, centred


def _random_pairs(n, seed):
    """Pairs built directly: rotated conics with axes of 0.3-3 voxels (log-
    uniform; half of them 0.3-0.8), centres within 7 voxels of the tile
    centre, t2 in [-40, -14]:
    many land near the chains' qualification bounds, where a wrong span or K
    shows."""
    g = np.random.default_rng(seed)
    sig = np.exp(g.uniform(np.log(0.3), np.log(3.0), (n, 3)))
    sig[: n // 2] = np.exp(g.uniform(np.log(0.3), np.log(0.8), (n // 2, 3)))  # steep rows
    q, _ = np.linalg.qr(g.normal(size=(n, 3, 3)))
    Q = np.einsum("nij,nj,nkj->nik", q, 1.0 / sig ** 2, q)
    con = np.stack([Q[:, 0, 0], Q[:, 0, 1], Q[:, 0, 2], Q[:, 1, 1], Q[:, 1, 2], Q[:, 2, 2]], 1)
    P = np.concatenate([g.uniform(-7, 7, (n, 3)), con.astype(np.float32),
                        g.uniform(-40, -14, (n, 1))], 1)
    return P.astype(np.float32).astype(np.float64)


def _needle_pairs(n, seed):
    """Tilted needles: one long axis (1.2-3 voxels) within 0.05-0.35 rad of x,
    two short ones (0.12-0.3 voxels).  Their conics couple x strongly to y and
    z (large |b|, |c| against a small a): the x-slope S1 of a row varies by far
    more over the tile than over the gate ellipse, and on rows away from the
    ellipse it can exceed 128, where 2^-S1 overflows binary32."""
    g = np.random.default_rng(seed)
    th = g.uniform(0.05, 0.35, n)
    ph = g.uniform(0, 2 * np.pi, n)
    u = np.stack([np.cos(th), np.sin(th) * np.cos(ph), np.sin(th) * np.sin(ph)], 1)
    v = np.cross(u, g.normal(size=(n, 3)))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    w = np.cross(u, v)
    R = np.stack([u, v, w], 2)                                    # columns: axes
    sig = np.stack([g.uniform(1.2, 3.0, n), g.uniform(0.12, 0.3, n), g.uniform(0.12, 0.3, n)], 1)
    Q = np.einsum("nij,nj,nkj->nik", R, 1.0 / sig ** 2, R)
    con = np.stack([Q[:, 0, 0], Q[:, 0, 1], Q[:, 0, 2], Q[:, 1, 1], Q[:, 1, 2], Q[:, 2, 2]], 1)
    P = np.concatenate([g.uniform(-6, 6, (n, 3)), con.astype(np.float32),
                        g.uniform(-40, -14, (n, 1))], 1)
    return P.astype(np.float32).astype(np.float64)


def _narrow():
    cfg = small_config(1, 3000, vol=(48, 56, 40))
    work = S.make_gaussians(cfg, seed=21)
    g = np.random.default_rng(22)
    vs = np.array([cfg.world[2] / cfg.vol[2], cfg.world[1] / cfg.vol[1], cfg.world[0] / cfg.vol[0]])
    s = np.exp(g.uniform(np.log(0.15), np.log(0.6), (cfg.n, 3))) * vs
    work.scale3d[:] = work.scale3d.new_tensor(s.astype(np.float32))
    return work


# (scene, sample of pairs, least share of them that must qualify: narrow
# Gaussians have steep rows, and few of their pairs take the chains)
SCENES = [
    ("cfg1", lambda: S.make_gaussians(S.CONFIGS[1], seed=0), 2500, 0.5),
    ("narrow", _narrow, 2500, 0.02),
    ("cfg5_mixture", lambda: S.make_gaussians(S.CONFIGS[5], seed=0, n=20000), 1500, 0.5),
    ("random_conics", None, 12000, 0.2),
]


@pytest.mark.parametrize("name,make,npairs,share", SCENES, ids=[s[0] for s in SCENES])
def test_chained_rows_gate_like_exp2(name, make, npairs, share):
    P = _random_pairs(npairs, seed=5) if make is None else _pairs(make(), npairs, seed=3)
    s_exact = _exact_exponent(P)
    fwd, fwd_ok = _forward_chains(P)
    n_f, live_f = _check(f"{name} forward", s_exact, fwd, fwd_ok)
    # the backward walks the same rows with the Gaussian-centred form
    bwd, bwd_ok, _, _ = _backward_chains(P)
    n_b, live_b = _check(f"{name} backward", s_exact, bwd, bwd_ok)
    assert n_f > share * len(P) and n_b > share * len(P), (name, n_f, n_b, len(P))
    assert live_f > 0 and live_b > 0


def test_backward_chain_bounds_dead_rows():
    """chain_shift's dead-row conditions (every tile row's slope |R1| below
    120, and the bound on E over the tile): pairs whose passing rows qualify
    but whose tile reaches beyond those bounds must take another path, and
    every qualifying pair stays finite with the right gate.  On rotated
    anisotropic conics and tilted needles; evaluated anyway, some of the
    excluded pairs overflow."""
    P = np.concatenate([_random_pairs(12000, seed=5), _needle_pairs(6000, seed=9)])
    s_exact = _exact_exponent(P)
    bwd, ok, excluded, centred = _backward_chains(P)
    n_b, live_b = _check("conics and needles backward", s_exact, bwd, ok)
    assert n_b > 0.3 * len(P) and live_b > 0, (n_b, len(P))
    # the scene exercises the conditions: without them these pairs would take
    # the chains and some of their products would overflow
    assert excluded.sum() > 0.01 * len(P), int(excluded.sum())
    assert not np.isfinite(bwd[excluded]).all()


def test_backward_ellipse_bound_in_binary32():
    """chain_shift's slope bound over the gate ellipse, sqrt(k2 w^T Q^-1 w) with
    w = (0, Bn, Cn), from a binary32 Cholesky factor of the conic: wherever both
    pivots stay above 1e-3 of their diagonal it agrees with the binary64
    cofactor formula to 2e-4 relative (the kernel's margin is 1e-3 + 0.01), on
    random rotated conics, narrow ones and tilted needles."""
    P = np.concatenate([_random_pairs(12000, seed=15), _needle_pairs(6000, seed=16)])
    F = np.float32
    ca, cb, cc_, cd, ce, cf = (P[:, 3 + i].astype(F) for i in range(6))
    t2 = P[:, 9].astype(F)
    Bn, Cn = F(-L2E) * cb, F(-L2E) * cc_
    k2 = (F(-2.0 * 0.693147180559945309) * t2).astype(F)
    with np.errstate(divide="ignore", invalid="ignore"):
        i11 = (F(1) / np.sqrt(ca)).astype(F)
        l21, l31 = cb * i11, cc_ * i11
        t22 = (cd - l21 * l21).astype(F)
        i22 = (F(1) / np.sqrt(t22)).astype(F)
        l32 = ((ce - l31 * l21) * i22).astype(F)
        t33 = (cf - l31 * l31 - l32 * l32).astype(F)
        y2 = Bn * i22
        y3 = ((Cn - l32 * y2) / np.sqrt(t33)).astype(F)
        got = np.sqrt(np.maximum(k2 * (y2 * y2 + y3 * y3), F(0))).astype(np.float64)
    ok = (t22 > F(1e-3) * cd) & (t33 > F(1e-3) * cf)
    a, b, c, d, e, f = (v.astype(np.float64) for v in (ca, cb, cc_, cd, ce, cf))
    syy, szz, syz = a * f - c * c, a * d - b * b, b * c - a * e
    det = a * (d * f - e * e) - b * (b * f - c * e) + c * (b * e - c * d)
    gb, gc = Bn.astype(np.float64), Cn.astype(np.float64)
    ref = np.sqrt(np.maximum(k2.astype(np.float64) *
                             (gb * gb * syy + 2 * gb * gc * syz + gc * gc * szz) / det, 0))
    assert ok.mean() > 0.9, ok.mean()
    rel = np.abs(got[ok] - ref[ok]) / np.maximum(ref[ok], 1e-30)
    assert rel.max() <= 2e-4, rel.max()
