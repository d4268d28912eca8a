"""HIP voxelization forward/backward against the oracle.

Bar (north_star): volume and gradients within rel 1e-4 / abs 1e-6 in fp32, on
the training gradient the benchmarks use (L1 loss against a phantom) and on a
harder seeded N(0,1) vol_grad where sums cancel.  Gradients add a
conditioning term: 1e-5 times the sum of |terms| of that element (reported by
the oracle), the summation-order error any binary32 evaluation can incur over
up to ~10^5 terms; it matters for elements that are small differences of large
sums (e.g. a Gaussian spanning hundreds of tiles, reduced with float atomics).

Every comparison also allows, per element, the oracle-reported magnitude of the
gate-ambiguous terms: evaluations whose alpha*mean lies within 1e-4 (relative)
of the 1e-6 threshold, or whose |sigma| < 1e-5.  Whether such a term counts is
decided by the last bits of binary32 rounding, so two correct fp32 evaluation
orders (and the reference's fast-math build) legitimately disagree on it.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import synthetic as S
from helpers import gpu_bin, l1_vol_grad, np32, oracle_project, report_close, small_config

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-6


def _prepare(work, device):
    """Project + bin on the GPU and cross-check the intermediates with the oracle."""
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    n = work.pos3d.shape[0]
    w = work.to(device)
    pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(n, w.pos3d, w.scale3d, w.quat,
                                                        w.intensities, cfg.vol, cfg.world,
                                                        cfg.center)
    cum, I, ids, bins = gpu_bin(n, tmin, tmax, nt, cfg.vol)
    rpr, rcn, rtmin, rtmax, rnt = oracle_project(work)
    rcum = O.cumsum(rnt)
    rids, rbins = O.bin_and_sort(n, int(rcum[-1]), rtmin, rtmax, rcum, cfg.vol)
    np.testing.assert_array_equal(np32(ids), rids)
    np.testing.assert_array_equal(np32(bins), rbins)
    return dict(w=w, pr=pr, cn=cn, I=I, ids=ids, bins=bins, rpr=rpr, rcn=rcn, rids=rids,
                rbins=rbins, tmin=tmin, tmax=tmax, cum=cum)


def _fwd_cases():
    yield "cfg1", S.make_gaussians(S.CONFIGS[1], seed=0)
    for c in (2, 3, 4):
        cfg = small_config(1, 3000, channels=c, world=(1.0, 1.5, 0.8), center=(0.5, 0.7, 0.5))
        yield f"multichannel_c{c}", S.make_gaussians(cfg, seed=c)
    yield "edge_tiles", S.make_gaussians(small_config(1, 800, vol=(20, 30, 17)), seed=8)
    yield "cfg2_20k", S.make_gaussians(small_config(2, 20000), seed=1)
    yield "cfg5_clustered_c4_8k", S.make_gaussians(small_config(5, 8000, vol=(64, 64, 64)), seed=9)
    # ~290 pairs per tile: the dense backward kernels at C = 2 and 3 (the small
    # multichannel scenes above, ~12 pairs per tile, take the sparse ones)
    for c in (2, 3):
        cfg = small_config(1, 6000, channels=c, vol=(40, 48, 40))
        yield f"dense_c{c}", S.make_gaussians(cfg, seed=20 + c)
    # ~46 pairs per tile: the middle staging tier of C > 1
    yield "mid_c3", S.make_gaussians(small_config(1, 3000, channels=3, vol=(64, 64, 64)), seed=31)


@pytest.mark.parametrize("name,work", list(_fwd_cases()), ids=lambda v: v if isinstance(v, str) else "")
def test_forward_matches_oracle(device, name, work):
    import gs_voxelizer.cuda as _C
    cfg = work.cfg
    P = _prepare(work, device)
    vol = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], P["w"].intensities)
    torch.cuda.synchronize()
    ref, amb = O.voxelize_fwd(cfg.vol, P["rids"], P["rbins"], P["rpr"], P["rcn"],
                              work.intensities.numpy(), with_amb=True)
    assert vol.shape == ref.shape
    report_close(f"{name}: volume", np32(vol), ref, RTOL, ATOL, bound=amb)


def test_forward_cfg3_full_size_tile_slab(device):
    """Headline size: every voxel of the first 2 z-layers of tiles (2048 tiles)."""
    import gs_voxelizer.cuda as _C
    work = S.make_gaussians(S.CONFIGS[3], seed=0)
    cfg = work.cfg
    P = _prepare(work, device)
    vol = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], P["w"].intensities)
    Tx, Ty, Tz = O.tile_grid(cfg.vol)
    t1 = 2 * Tx * Ty
    ref, amb = O.voxelize_fwd(cfg.vol, P["rids"], P["rbins"], P["rpr"], P["rcn"],
                              work.intensities.numpy(), tile_range=(0, t1), with_amb=True)
    report_close("cfg3 slab volume", np32(vol[:16]), ref[:16], RTOL, ATOL, bound=amb[:16])
    assert float(vol[16:].abs().sum()) > 0


MODES = ["pairs", "atomic"]  # deterministic per-pair reduction / float atomics


def _gpu_bwd(P, cfg, g, variant=1, mode="pairs"):
    import gs_voxelizer.cuda as _C
    fn = _C.voxelize_backward_per_gaussian if variant == 1 else _C.voxelize_backward
    extra = (P["tmin"], P["tmax"], P["cum"]) if mode == "pairs" else ()
    return fn(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], P["w"].intensities, g, *extra)


def _bwd(work, device, vol_grad_np, variant=1, mode="pairs"):
    cfg = work.cfg
    P = _prepare(work, device)
    g = torch.from_numpy(vol_grad_np).to(device)
    dp, dc, di = _gpu_bwd(P, cfg, g, variant, mode)
    torch.cuda.synchronize()
    ref, absum, amb = O.voxelize_bwd(cfg.vol, P["rids"], P["rbins"], P["rpr"], P["rcn"],
                                     work.intensities.numpy(), vol_grad_np, diagnostics=True)
    return P, (np32(dp), np32(dc), np32(di)), ref, absum, amb


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("name,work", list(_fwd_cases()), ids=lambda v: v if isinstance(v, str) else "")
def test_backward_l1_gradient_matches_oracle(device, name, work, mode):
    """The benchmark's gradient: L1 loss against the config's phantom."""
    cfg = work.cfg
    P = _prepare(work, device)
    ref_vol = O.voxelize_fwd(cfg.vol, P["rids"], P["rbins"], P["rpr"], P["rcn"],
                             work.intensities.numpy())
    target = S.phantom(work).numpy()[..., None]
    g = l1_vol_grad(ref_vol, np.broadcast_to(target, ref_vol.shape))
    _, got, ref, absum, amb = _bwd(work, device, g, mode=mode)
    for nm, a, b, s, m in zip(("dpos3d_radii", "dconics", "dintensities"), got, ref, absum, amb):
        report_close(f"{name}: {nm}", a, b, RTOL, ATOL, bound=1e-5 * s + m)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("name,work", list(_fwd_cases())[:5] + list(_fwd_cases())[-3:],
                         ids=lambda v: v if isinstance(v, str) else "")
def test_backward_random_gradient_conditioned(device, name, work, mode):
    cfg = work.cfg
    C = work.intensities.shape[1]
    g = np.random.default_rng(5).standard_normal(cfg.vol + (C,)).astype(np.float32)
    _, got, ref, absum, amb = _bwd(work, device, g, mode=mode)
    for nm, a, b, s, m in zip(("dpos3d_radii", "dconics", "dintensities"), got, ref, absum, amb):
        report_close(f"{name}: {nm}", a, b, RTOL, ATOL, bound=1e-5 * s + m)


def test_backward_variants_agree(device):
    work = S.make_gaussians(S.CONFIGS[1], seed=2)
    g = np.random.default_rng(1).standard_normal(work.cfg.vol + (1,)).astype(np.float32)
    _, got1, _, absum, _ = _bwd(work, device, g, variant=1, mode="atomic")
    _, got0, _, _, _ = _bwd(work, device, g, variant=0, mode="atomic")
    for nm, a, b, s in zip(("dpos3d_radii", "dconics", "dintensities"), got0, got1, absum):
        report_close(f"variants {nm}", a, b, 1e-6, 0.0, bound=1e-6 * s)


def test_backward_pairs_bitwise_reproducible(device):
    """The per-pair reduction has a fixed summation order: two runs, and both
    variants, give identical bits; atomics agree with it to rounding."""
    work = S.make_gaussians(small_config(3, 40000, vol=(96, 128, 80)), seed=6)
    cfg = work.cfg
    P = _prepare(work, device)
    g = torch.randn(cfg.vol + (1,), generator=torch.Generator().manual_seed(2)).to(device)
    a = [t.cpu() for t in _gpu_bwd(P, cfg, g, 1, "pairs")]
    b = [t.cpu() for t in _gpu_bwd(P, cfg, g, 1, "pairs")]
    c = [t.cpu() for t in _gpu_bwd(P, cfg, g, 0, "pairs")]
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y) and torch.equal(x, z)
    d = [t.cpu().numpy() for t in _gpu_bwd(P, cfg, g, 1, "atomic")]
    for nm, x, y in zip(("dpos3d_radii", "dconics", "dintensities"), a, d):
        scale = float(np.abs(y).max())
        report_close(f"pairs vs atomic {nm}", x.numpy(), y, 1e-4, 1e-5 * scale)


def test_backward_cfg3_full_size_identity(device):
    """Full headline size, size-independent check: for one channel the volume is
    linear in the intensities, so sum_g I_g * dL/dI_g == sum_v vol_v * g_v."""
    import gs_voxelizer.cuda as _C
    work = S.make_gaussians(S.CONFIGS[3], seed=0)
    cfg = work.cfg
    P = _prepare(work, device)
    I = P["w"].intensities
    vol = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"], I)
    gen = torch.Generator(device="cpu").manual_seed(3)
    g = torch.randn(vol.shape, generator=gen).to(device)
    dp, dc, di = _C.voxelize_backward_per_gaussian(cfg.vol, P["ids"], P["bins"], P["pr"], P["cn"],
                                                   I, g, P["tmin"], P["tmax"], P["cum"])
    lhs = float((I.double() * di.double()).sum())
    rhs = float((vol.double() * g.double()).sum())
    scale = float((vol.double() * g.double()).abs().sum())
    assert abs(lhs - rhs) <= 1e-5 * scale, (lhs, rhs, scale)
    assert torch.isfinite(dp).all() and torch.isfinite(dc).all() and torch.isfinite(di).all()
    assert float(dp[:, 3].abs().sum()) == 0.0


def _mixed_gate_inputs(work, P):
    """Gaussians outside the gate-free domain, interleaved in the same tiles
    (and backward waves) with ordinary ones: indefinite conics, means beyond
    2^60 * 1e-6, channels spread far beyond their mean, and means below 1e-6."""
    rng = np.random.default_rng(12)
    n = work.pos3d.shape[0]
    pr, cn = P["rpr"].copy(), P["rcn"].copy()
    inten = work.intensities.numpy().copy()
    k = rng.permutation(n)
    indef, huge, spread, dead = k[:60], k[60:80], k[80:120], k[120:140]
    cn[indef, 5] = -0.05 * np.abs(cn[indef, 5])  # negative zz entry: indefinite form
    inten[huge] *= np.float32(1e14)               # log2(1e-6 / mean) < -60
    if inten.shape[1] > 1:
        inten[spread, 0] = 3e7                    # mean ~0.5, |I| ~ 2^25 * mean
        inten[spread, 1] = -3e7 + 4  # binary32 spacing at 3e7 is 2: mean 2 exactly
    inten[dead] = 5e-7                            # alpha * mean < 1e-6 everywhere
    return pr, cn, inten


@pytest.mark.parametrize("channels", [2, 1])
def test_mixed_gate_paths_match_oracle(device, channels):
    """Exact-gate Gaussians sharing tiles with gate-free ones, forward and both
    backward reductions.  At C = 1 the forward accumulates in units of
    1e-6 * 2^126 on every path, the exact one included."""
    import gs_voxelizer.cuda as _C
    cfg = small_config(1, 1500, vol=(24, 32, 28), channels=channels)
    work = S.make_gaussians(cfg, seed=12)
    P = _prepare(work, device)
    pr, cn, inten = _mixed_gate_inputs(work, P)
    dpr, dcn, dI = (torch.from_numpy(x).to(device) for x in (pr, cn, inten))
    vol = _C.voxelize_forward(cfg.vol, P["ids"], P["bins"], dpr, dcn, dI)
    ref, amb = O.voxelize_fwd(cfg.vol, P["rids"], P["rbins"], pr, cn, inten, with_amb=True)
    # Signed channels of magnitude 3e7 cancel to ~1e4 here, so the forward gets
    # the conditioning term the gradients have.  The oracle on |I| bounds the sum
    # of |terms| from above: mean(|I|) >= mean(I) only lowers the threshold.
    cond = O.voxelize_fwd(cfg.vol, P["rids"], P["rbins"], pr, cn, np.abs(inten))
    report_close("mixed gates: volume", np32(vol), ref, RTOL, ATOL, bound=amb + 1e-5 * cond)
    g = np.random.default_rng(3).standard_normal(cfg.vol + (channels,)).astype(np.float32)
    rg, absum, ramb = O.voxelize_bwd(cfg.vol, P["rids"], P["rbins"], pr, cn, inten, g,
                                     diagnostics=True)
    for mode in MODES:
        extra = (P["tmin"], P["tmax"], P["cum"]) if mode == "pairs" else ()
        got = _C.voxelize_backward_per_gaussian(cfg.vol, P["ids"], P["bins"], dpr, dcn, dI,
                                                torch.from_numpy(g).to(device), *extra)
        for nm, a, b, s, m in zip(("dpos3d_radii", "dconics", "dintensities"), got, rg, absum,
                                  ramb):
            report_close(f"mixed gates {mode}: {nm}", np32(a), b, RTOL, ATOL, bound=1e-5 * s + m)


@pytest.mark.parametrize("e", [-60, 60])
def test_backward_power_of_two_gradient_scaling_is_exact(device, e):
    """The gradients are linear in vol_grad.  Scaling vol_grad by 2^e must scale
    every gradient by exactly 2^e, bit for bit: the kernel stages each tile's
    vol_grad with its own power-of-two scale, so tiny loss gradients (where
    alpha * g would otherwise be denormal) lose nothing."""
    work = S.make_gaussians(small_config(2, 6000, vol=(64, 64, 64)), seed=4)
    cfg = work.cfg
    P = _prepare(work, device)
    g = torch.randn(cfg.vol + (1,), generator=torch.Generator().manual_seed(7)).to(device)
    base = [t.cpu() for t in _gpu_bwd(P, cfg, g, 1, "pairs")]
    scaled = [t.cpu() for t in _gpu_bwd(P, cfg, torch.ldexp(g, torch.tensor(float(e))), 1,
                                        "pairs")]
    for x, y in zip(base, scaled):
        assert torch.equal(torch.ldexp(x, torch.tensor(float(e))), y)
    assert float(base[2].abs().sum()) > 0


# A tilted needle (one long axis near x, two of ~0.15 voxel) whose rows inside
# its gate ellipse admit the backward's chained rows (3M + 2 = 76 <= K = 95),
# while on rows of its tile away from the ellipse the x-slope reaches
# m_tile = 145: there 2^-S1 overflows binary32.  Found with the CPU restatement
# of the chains in test_chain_cpu.py (needle scene, seed 9, pair 2300):
# centre offset from the tile centre, conic (00, 01, 02, 11, 12, 22), and
# t2 = log2(1e-6 / I).
_NEEDLE = np.array([3.490655, 1.9826925, -3.301888, 2.745941, 9.987584, -5.312871, 52.159576,
                    -15.002705, 25.211243, -14.04277], np.float32)


def test_backward_chain_guard_on_needle_in_a_chained_wave(device):
    """One tile, one backward wave: 63 round Gaussians that take the chained
    rows and the needle above.  Chained anyway, the needle's dead rows would
    turn into inf / NaN (the CPU restatement of the chain shows it); chain_shift
    refuses it, so the wave takes another path, and every gradient matches the
    oracle."""
    import gs_voxelizer.cuda as _C
    from test_chain_cpu import _backward_chains
    P = _NEEDLE.astype(np.float64)[None, :]
    chained, qualifies, _, _ = _backward_chains(P)
    assert not qualifies[0] and not np.isfinite(chained).all()
    rng = np.random.default_rng(1)
    n, vol, centre = 64, (24, 24, 24), np.float32(12.0)  # tile (1, 1, 1): voxels 8..15
    pr = np.zeros((n, 4), np.float32)
    cn = np.zeros((n, 6), np.float32)
    inten = np.full((n, 1), 0.5, np.float32)
    sig = rng.uniform(1.0, 2.0, n - 1)
    pr[:-1, :3] = centre + rng.uniform(-3, 3, (n - 1, 3))
    pr[:, 3] = 3.0
    cn[:-1, 0] = cn[:-1, 3] = cn[:-1, 5] = 1.0 / sig ** 2
    pr[-1, :3] = centre + _NEEDLE[:3]
    cn[-1] = _NEEDLE[3:9]
    inten[-1, 0] = np.float32(2.0 ** (np.log2(1e-6) - float(_NEEDLE[9])))
    tmin = np.ones((n, 3), np.int32)
    tmax = np.full((n, 3), 2, np.int32)
    nt = np.ones(n, np.int32)
    cum = O.cumsum(nt)
    rids, rbins = O.bin_and_sort(n, n, tmin, tmax, cum, vol)
    g = rng.standard_normal(vol + (1,)).astype(np.float32)
    ref, absum, amb = O.voxelize_bwd(vol, rids, rbins, pr, cn, inten, g, diagnostics=True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    ids, bins = _C.bin_and_sort_gaussians(n, n, t(tmin), t(tmax), t(cum), vol)
    for mode in MODES:
        extra = (t(tmin), t(tmax), t(cum)) if mode == "pairs" else ()
        got = _C.voxelize_backward_per_gaussian(vol, ids, bins, t(pr), t(cn), t(inten), t(g),
                                                *extra)
        torch.cuda.synchronize()
        for nm, a, b, s, m in zip(("dpos3d_radii", "dconics", "dintensities"), got, ref, absum,
                                  amb):
            a = np32(a)
            assert np.isfinite(a).all(), f"needle {mode}: {nm} not finite"
            report_close(f"needle guard {mode}: {nm}", a, b, RTOL, ATOL, bound=1e-5 * s + m)


@pytest.mark.parametrize("mode", MODES)
def test_backward_gaussians_without_pairs_get_zero_gradients(device, mode):
    """A Gaussian with no (tile, Gaussian) pair gets zero gradients in both
    reduction modes, whatever its conic holds: the per-pair mode applies each
    Gaussian's conic once, to the sum of its pairs' moments, and only when it
    has pairs.  The other Gaussians' gradients do not depend on those conics."""
    work = S.make_gaussians(S.CONFIGS[1], seed=0)
    outside = torch.arange(0, 40, 5)
    work.pos3d[outside] = 5.0  # far outside the [0, 1]^3 world box: no tiles
    cfg = work.cfg
    P = _prepare(work, device)
    nt = np.diff(np.concatenate([[0], np32(P["cum"]).astype(np.int64)]))
    assert (nt[outside.numpy()] == 0).all() and (nt > 0).sum() > 1000
    C = work.intensities.shape[1]
    g = torch.from_numpy(np.random.default_rng(3).standard_normal(cfg.vol + (C,)).astype(np.float32))
    g = g.to(device)
    base = [np32(t) for t in _gpu_bwd(P, cfg, g, 1, mode)]
    cn = P["cn"].clone()
    cn[outside[::2].to(device)] = float("inf")
    cn[outside[1::2].to(device)] = float("nan")
    P2 = dict(P, cn=cn)
    got = [np32(t) for t in _gpu_bwd(P2, cfg, g, 1, mode)]
    torch.cuda.synchronize()
    rest = np.ones(nt.shape[0], bool)
    rest[outside.numpy()] = False
    for nm, a, b in zip(("dpos3d_radii", "dconics", "dintensities"), got, base):
        assert (a[outside.numpy()] == 0).all(), nm
        if mode == "pairs":  # float atomics leave the last bits to the schedule
            np.testing.assert_array_equal(a[rest], b[rest], err_msg=nm)
