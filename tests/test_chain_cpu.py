"""The chained row evaluation of the voxelize kernels, checked on the CPU.

Both voxelize kernels form most exp2 values of an 8-voxel row as products
(an anchor 2^E and a step along the row, times per-pair column factors:
2^(A2 uc^2 - K) about the tile centre in the forward, 2^(-x_u^2 - K) in the
backward's row form, the LDL^T coordinates of the conic about the tile centre)
and rely on binary32 flush-to-zero for
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


def _row_form(P):
    """row_form (csrc/voxelize.hip) per pair: the binary64 LDL^T factor of the
    conic and the row-form coefficients about the tile centre, rounded to
    binary32 as the kernel rounds them.  Returns (ok, al, be, ga, be2, ga2,
    ga3, tc, ec, zc, r_ell)."""
    F = np.float32
    mx, my, mz = (P[:, i].astype(F).astype(np.float64) for i in range(3))
    a, b, c, d, e, f = (P[:, 3 + i].astype(F).astype(np.float64) for i in range(6))
    k = 0.5 * L2E
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        l21, l31 = b / a, c / a
        d2, e2, f2 = d - b * l21, e - c * l21, f - c * l31
        l32 = e2 / d2
        d3 = f2 - e2 * l32
        p1, p2, p3 = k * a, k * d2, k * d3
        ok = np.ones(len(P), bool)
        for pv in (p1, p2, p3):
            ok &= (pv >= 2.0 ** -100) & (pv <= 2.0 ** 100)
        al = np.sqrt(p1.astype(F)).astype(np.float64)
        b2 = np.sqrt(p2.astype(F)).astype(np.float64)
        g3 = np.sqrt(p3.astype(F)).astype(np.float64)
        y2 = 2.0 * k * b
        y3 = 2.0 * k * c - l32 * y2
        r_ell = y2 * y2 / d2 + y3 * y3 / d3
        out = (al, al * l21, al * l31, b2, b2 * l32, g3, al * (mx + l21 * my + l31 * mz),
               b2 * (my + l32 * mz), g3 * mz.astype(F), r_ell)
    z = F(0)
    out = tuple(np.where(ok, _f(v), z).astype(F) for v in out)
    return (ok,) + out


def _backward_chains(P):
    """The backward's rows (lane = pair, rows walked in order), as pair_moments
    with kRowsChain forms them from the row form (LDL^T coordinates of the
    conic about the tile centre): a_u = 2^E_u * G_u with E_u = q_r + 2 u_r x_u
    (q_r = c_r - u_r^2, c_r holding off + K) at the anchors u = 0 and u = 4,
    each stepped three times by 2^(2 al u_r), times the column factors
    G_u = 2^(-x_u^2 - K) at the positions the chain implies (x_a + (u - a) al,
    the square in binary64 with its binary32 residual); and chain_shift's K.
    Returns (a, qualifies, excluded, K): excluded are the pairs whose rows that
    can hold a passing voxel qualify but whose tile's other rows exceed the
    slope bound (m_tile >= 120); their rows are evaluated with that K anyway."""
    uc, py, pz = _grid()
    F = np.float32
    mx = P[:, 0].astype(F)
    ca = P[:, 3].astype(F)
    t2 = P[:, 9].astype(F)
    off = (-(t2 + F(126.0))).astype(F)
    ok, al, be, ga, be2, ga2, ga3, tc, ec, zc, r_ell = _row_form(P)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        a2 = _f(al * al)
        k2 = (F(-2.0 * 0.693147180559945309) * t2).astype(F)
        m_tile = _f(F(2.0) * al * _f(np.abs(tc) + F(3.5) * (np.abs(be) + np.abs(ga))))
        k_max = np.floor(F(120.0) - F(12.25) * a2).astype(F)
        m_reach = _f(F(2.0) * a2 * _f(F(3.5) + np.sqrt(np.maximum(k2 / ca, F(0))).astype(F)))
        m_ell = _f(F(2.0) * a2 * np.abs(mx) + np.sqrt(np.maximum(k2 * r_ell, F(0))).astype(F))
        m_rows = np.minimum(m_ell, m_reach)
        M = _f(np.minimum(m_tile, m_rows) * F(1.001) + F(0.01))
        k_min = (np.ceil(F(3.0) * M) + 2).astype(F)
        rows_ok = ok & (np.ceil(F(3.0) * _f(m_rows * F(1.001) + F(0.01))) + 2 <= k_max)
        qualifies = ok & (m_tile < F(120.0)) & (k_min <= k_max)
        K = np.minimum(k_max, np.maximum(k_min, np.rint(-off))).astype(F)
        K = np.where(qualifies, K, np.maximum(k_max, F(2.0))).astype(F)
    excluded = rows_ok & ~(m_tile < F(120.0))
    xu = _f(al[:, None] * uc[None, :].astype(F))                       # (N, 8)
    anc = xu[:, [0, 0, 0, 0, 4, 4, 4, 4]].astype(np.float64)
    xe = anc + al[:, None].astype(np.float64) * np.array([0, 1, 2, 3, 0, 1, 2, 3])
    d = -xe * xe
    hi = _f(d)
    lo = _f(d - hi.astype(np.float64))
    with np.errstate(over="ignore"):
        G = _ftz(np.ldexp(np.float64(_f(np.float64(_exp2(hi)) *
                                         _fma(lo, F(0.693147180559945309), F(1)))),
                          -K.astype(np.int64)[:, None]))
    c0 = _f(off + K)
    al2 = _f(F(2.0) * al)
    out = np.zeros((P.shape[0], 64, 8), np.float32)
    for lz in range(8):
        pzl = F(lz - 3.5)
        zt = _fma(-ga3, pzl, zc)
        zz = _fma(-zt, zt, c0)
        tz = _fma(-ga, pzl, tc)
        ez = _fma(-ga2, pzl, ec)
        for ly in range(8):
            row = lz * 8 + ly
            pyl = F(ly - 3.5)
            ur = _fma(-be, pyl, tz)
            et = _fma(-be2, pyl, ez)
            cr = _fma(-et, et, zz)
            q = _fma(-ur, ur, cr)
            step = _exp2(_f(ur * al2))
            e1 = _exp2(_fma(ur, _f(F(2.0) * xu[:, 0]), q))
            e2 = _exp2(_fma(ur, _f(F(2.0) * xu[:, 4]), q))
            for k in range(4):
                out[:, row, k] = _mul(e1, G[:, k])
                out[:, row, 4 + k] = _mul(e2, G[:, 4 + k])
                e1, e2 = _mul(e1, step), _mul(e2, step)
    return out, qualifies, excluded, K


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
    # the backward walks the same rows with its row form
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
    bwd, ok, excluded, _ = _backward_chains(P)
    n_b, live_b = _check("conics and needles backward", s_exact, bwd, ok)
    assert n_b > 0.3 * len(P) and live_b > 0, (n_b, len(P))
    # the scene exercises the conditions: without them these pairs would take
    # the chains and some of their products would overflow
    assert excluded.sum() >= 100, int(excluded.sum())
    assert not np.isfinite(bwd[excluded]).all()


def test_backward_row_form_is_the_quadratic_form():
    """row_form's LDL^T coordinates: -(tau^2 + eta^2 + zeta^2), from the
    binary32-rounded coefficients exactly as the kernel combines them, equals
    sigma2 = -log2(e)/2 * delta^T Q delta for every voxel of the tile to
    within 5e-6 of the larger of |sigma2| and 1 (the binary32 rounding of
    coefficients of up to ~10 that multiply |p'| <= 3.5), and r_ell equals w^T Q^-1 w
    (w = log2(e) (0, b, c)) from the binary64 cofactors to 1e-6 relative; on
    rotated anisotropic conics and tilted needles."""
    P = np.concatenate([_random_pairs(6000, seed=15), _needle_pairs(3000, seed=16)])
    ok, al, be, ga, be2, ga2, ga3, tc, ec, zc, r_ell = (np.asarray(v, np.float64)
                                                         for v in _row_form(P))
    ok = ok.astype(bool)
    assert ok.mean() > 0.99, ok.mean()
    uc, py, pz = _grid()
    tau = tc[:, None, None] - al[:, None, None] * uc[None, None, :] - \
        (be[:, None] * py[None, :] + ga[:, None] * pz[None, :])[:, :, None]
    eta = (ec[:, None] - be2[:, None] * py[None, :] - ga2[:, None] * pz[None, :])[:, :, None]
    zeta = (zc[:, None] - ga3[:, None] * pz[None, :])[:, :, None]
    got = -(tau * tau + eta * eta + zeta * zeta)
    t2 = P[:, 9]
    want = _exact_exponent(P) + (t2 + 126.0)[:, None, None]      # sigma2 alone
    err = np.abs(got - want) / np.maximum(np.abs(want), 1.0)
    assert err[ok].max() <= 5e-6, err[ok].max()
    a, b, c, d, e, f = (P[:, 3 + i].astype(np.float32).astype(np.float64) for i in range(6))
    syy, szz, syz = a * f - c * c, a * d - b * b, b * c - a * e
    det = a * (d * f - e * e) - b * (b * f - c * e) + c * (b * e - c * d)
    gb, gc = L2E * b, L2E * c
    ref = (gb * gb * syy + 2 * gb * gc * syz + gc * gc * szz) / det
    rel = np.abs(r_ell[ok] - ref[ok]) / ref[ok]
    assert rel.max() <= 1e-6, rel.max()
