"""Seeded synthetic workloads for the five benchmark configurations.

These play the role of the reference's test fixtures (test/utils.py:10-154:
random-sphere phantom, smoothed-noise phantom, random_gauss_init) with every
random draw taken from one CPU ``torch.Generator`` in a fixed order
(positions, scales, quaternions, intensities, phantom), so the GPU run and any
CPU check see bit-identical inputs.

Conventions: positions are world units (x, y, z) in a world box of size
``world`` (z, y, x) centred at ``center`` (z, y, x); a scale of "s voxels"
on axis k means scale3d[:, k] = s * world_k / N_k.
"""
import math

import numpy as np
from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class Config:
    name: str
    vol: Tuple[int, int, int]              # (D, H, W)
    n: int
    channels: int
    scale: Tuple                           # ("axis"|"iso", lo, hi) or ("mixture",)
    quat: str                              # "random" | "identity"
    intensity: Tuple[float, float]
    position: str                          # "uniform" | "clustered"
    phantom: str                           # "smooth" | "ellipsoids"
    world: Tuple[float, float, float] = (1.0, 1.0, 1.0)
    center: Tuple[float, float, float] = (0.5, 0.5, 0.5)


CONFIGS: Dict[int, Config] = {
    1: Config("cfg1_readme_100x150x80_5k", (100, 150, 80), 5_000, 1, ("axis", 0.5, 4.0), "random",
              (0.0, 1.0), "uniform", "smooth"),
    2: Config("cfg2_128cube_50k", (128, 128, 128), 50_000, 1, ("iso", 0.5, 3.0), "identity",
              (0.0, 0.5), "uniform", "ellipsoids"),
    3: Config("cfg3_256cube_200k", (256, 256, 256), 200_000, 1, ("axis", 0.5, 6.0), "random",
              (0.0, 1.0), "uniform", "ellipsoids"),
    4: Config("cfg4_512cube_1M", (512, 512, 512), 1_000_000, 1, ("axis", 0.5, 8.0), "random",
              (0.0, 0.2), "uniform", "ellipsoids"),
    5: Config("cfg5_256cube_500k_c4", (256, 256, 256), 500_000, 4, ("mixture",), "random",
              (0.0, 1.0), "clustered", "ellipsoids"),
}


def _log_uniform(g, shape, lo, hi):
    u = torch.rand(shape, generator=g, dtype=torch.float64)
    return torch.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))


def voxel_size_xyz(cfg: Config) -> torch.Tensor:
    D, H, W = cfg.vol
    wz, wy, wx = cfg.world
    return torch.tensor([wx / W, wy / H, wz / D], dtype=torch.float64)


@dataclass
class Workload:
    cfg: Config
    pos3d: torch.Tensor
    scale3d: torch.Tensor
    quat: torch.Tensor
    intensities: torch.Tensor
    phantom_params: Optional[dict] = field(default=None)
    seed: int = 0

    def to(self, device):
        return Workload(self.cfg, self.pos3d.to(device), self.scale3d.to(device),
                        self.quat.to(device), self.intensities.to(device), self.phantom_params,
                        self.seed)


def make_gaussians(cfg: Config, seed: int = 0, n: Optional[int] = None) -> Workload:
    """Draw the Gaussians of ``cfg`` (optionally only the first ``n``) on the CPU."""
    n = cfg.n if n is None else int(n)
    g = torch.Generator(device="cpu").manual_seed(seed)
    # positions (world units, x y z)
    if cfg.position == "uniform":
        pos = torch.rand((n, 3), generator=g, dtype=torch.float64)
    else:  # 16-component isotropic normal mixture, sigma 0.05, centres U[0,1]^3, unclipped
        centres = torch.rand((16, 3), generator=g, dtype=torch.float64)
        comp = torch.randint(0, 16, (n,), generator=g)
        pos = centres[comp] + 0.05 * torch.randn((n, 3), generator=g, dtype=torch.float64)
    cz, cy, cx = cfg.center
    wz, wy, wx = cfg.world
    origin = torch.tensor([cx - wx / 2, cy - wy / 2, cz - wz / 2], dtype=torch.float64)
    extent = torch.tensor([wx, wy, wz], dtype=torch.float64)
    pos = origin + pos * extent
    # scales, in voxels, converted to world units per axis
    kind = cfg.scale[0]
    if kind == "axis":
        s = _log_uniform(g, (n, 3), cfg.scale[1], cfg.scale[2])
    elif kind == "iso":
        s = _log_uniform(g, (n, 1), cfg.scale[1], cfg.scale[2]).expand(n, 3)
    else:  # 90% LU[0.5,2], 10% LU[8,32] voxels, per axis
        big = torch.rand((n,), generator=g, dtype=torch.float64) < 0.1
        small_s = _log_uniform(g, (n, 3), 0.5, 2.0)
        big_s = _log_uniform(g, (n, 3), 8.0, 32.0)
        s = torch.where(big[:, None], big_s, small_s)
    scale = s * voxel_size_xyz(cfg)
    # rotations [w, x, y, z]
    if cfg.quat == "random":
        q = torch.randn((n, 4), generator=g, dtype=torch.float64)
        q = q / q.norm(dim=1, keepdim=True)
    else:
        q = torch.zeros((n, 4), dtype=torch.float64)
        q[:, 0] = 1.0
    lo, hi = cfg.intensity
    inten = lo + (hi - lo) * torch.rand((n, cfg.channels), generator=g, dtype=torch.float64)
    # phantom parameters (drawn last, so they do not perturb the Gaussians)
    params = {"kind": cfg.phantom}
    if cfg.phantom == "ellipsoids":
        k = 20
        params.update(
            centres=torch.rand((k, 3), generator=g, dtype=torch.float64),
            semi=0.05 + 0.15 * torch.rand((k, 3), generator=g, dtype=torch.float64),
            rot=torch.randn((k, 4), generator=g, dtype=torch.float64),
            value=0.5 + 0.5 * torch.rand((k,), generator=g, dtype=torch.float64))
    else:
        params.update(noise_seed=int(torch.randint(0, 2**31 - 1, (1,), generator=g)))
    return Workload(cfg, pos.float().contiguous(), scale.float().contiguous(),
                    q.float().contiguous(), inten.float().contiguous(), params, seed)


def _rotmat(q: torch.Tensor) -> torch.Tensor:
    q = q / q.norm(dim=-1, keepdim=True)
    w, x, y, z = q.unbind(-1)
    return torch.stack([
        torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], -2)


def phantom(work: Workload, device="cpu") -> torch.Tensor:
    """Target volume (D, H, W) float32 in [0, 1] (test/utils.py:10-71 analogues)."""
    cfg = work.cfg
    D, H, W = cfg.vol
    p = work.phantom_params
    if p["kind"] == "smooth":
        gn = torch.Generator(device="cpu").manual_seed(p["noise_seed"])
        noise = torch.rand((1, 1, D, H, W), generator=gn, dtype=torch.float32).to(device)
        vol = 0.1 + 0.9 * F.avg_pool3d(noise, kernel_size=5, stride=1, padding=2)
        return vol.clamp(0.0, 1.0)[0, 0].contiguous()
    wz, wy, wx = cfg.world
    cz, cy, cx = cfg.center
    vol = torch.full((D, H, W), 0.1, dtype=torch.float32, device=device)
    xs = (cx - wx / 2) + (torch.arange(W, device=device, dtype=torch.float32) + 0.5) * (wx / W)
    ys = (cy - wy / 2) + (torch.arange(H, device=device, dtype=torch.float32) + 0.5) * (wy / H)
    zs = (cz - wz / 2) + (torch.arange(D, device=device, dtype=torch.float32) + 0.5) * (wz / D)
    origin = torch.tensor([cx - wx / 2, cy - wy / 2, cz - wz / 2], dtype=torch.float64)
    extent = torch.tensor([wx, wy, wz], dtype=torch.float64)
    centres = (origin + p["centres"] * extent).float().to(device)
    R = _rotmat(p["rot"]).float().to(device)
    semi = p["semi"].float().to(device)
    val = p["value"].float().to(device)
    chunk = max(1, (1 << 24) // (H * W))
    for z0 in range(0, D, chunk):
        zz = zs[z0:z0 + chunk]
        P = torch.stack(torch.meshgrid(xs, ys, zz, indexing="ij"), -1)  # (W, H, dz, 3)
        acc = torch.zeros(P.shape[:3], dtype=torch.float32, device=device)
        for e in range(centres.shape[0]):
            d = (P - centres[e]) @ R[e]  # body-frame coordinates
            inside = ((d / semi[e]) ** 2).sum(-1) <= 1.0
            acc += inside.float() * val[e]
        vol[z0:z0 + chunk] += acc.permute(2, 1, 0)
    return vol.clamp_(0.0, 1.0)


def tile_grid(vol):
    D, H, W = vol
    return (W + 7) // 8, (H + 7) // 8, (D + 7) // 8


# The reference's own value scenario (test/test_gs_voxelizer.py:15-26): a
# (100, 150, 80) volume in a unit world centred at 0.5 and 100,000 Gaussians
# from random_gauss_init(anisotropicScale=True, rotation=True)
# (test/utils.py:91-154), intensities divided by 10.  The reference draws
# from unseeded global generators; here every draw comes from seeded ones.
REFERENCE_SCENARIO = Config("ref_value_test_100x150x80_100k", (100, 150, 80), 100_000, 1,
                            ("fixed", 0.03, 0.01, 0.02), "euler_xyz", (0.01, 0.1), "uniform",
                            "spheres")


def sphere_phantom(vol, rng) -> torch.Tensor:
    """generate_test_volume (test/utils.py:10-29) with a seeded numpy Generator:
    0.1 everywhere plus 20 balls, centres uniform over the voxel indices, radii
    uniform integers in [D // 10, D // 5), each adding U(0.5, 1) inside, then
    clipped to [0, 1].  (D, H, W) float32."""
    D, H, W = vol
    out = torch.full((D, H, W), 0.1, dtype=torch.float32)
    zz = torch.arange(D)[:, None, None]
    yy = torch.arange(H)[None, :, None]
    xx = torch.arange(W)[None, None, :]
    for _ in range(20):
        c = rng.integers(0, [D, H, W], size=3)
        r = int(rng.integers(max(1, D // 10), max(2, D // 5)))
        inside = (zz - int(c[0])) ** 2 + (yy - int(c[1])) ** 2 + (xx - int(c[2])) ** 2 <= r * r
        out[inside] += float(rng.uniform(0.5, 1.0))
    return out.clamp_(0.0, 1.0)


def reference_value_scenario(seed: int = 0, n: Optional[int] = None):
    """(Workload, phantom (D, H, W)) of the reference's value test, seeded.

    Positions U[0,1)^3 (world units, x y z); scales (0.02 * 1.5, 0.02 * 0.5,
    0.02) world units; rotations from XYZ Euler angles U[0, 360) degrees
    through the half-angle product formula; intensity = the phantom's value at
    the voxel floor(pos * (size - 1)) per axis, divided by 10, as
    random_gauss_init reads it in float32."""
    cfg = REFERENCE_SCENARIO
    n = cfg.n if n is None else int(n)
    D, H, W = cfg.vol
    vol = sphere_phantom(cfg.vol, np.random.default_rng(seed))
    g = torch.Generator(device="cpu").manual_seed(seed)
    pos = torch.rand((n, 3), generator=g, dtype=torch.float32)
    scale = torch.tensor([0.03, 0.01, 0.02], dtype=torch.float32).expand(n, 3).contiguous()
    half = torch.deg2rad(torch.rand((n, 3), generator=g, dtype=torch.float32) * 360) / 2
    c, s = torch.cos(half), torch.sin(half)
    quat = torch.stack([c[:, 0] * c[:, 1] * c[:, 2] + s[:, 0] * s[:, 1] * s[:, 2],
                        s[:, 0] * c[:, 1] * c[:, 2] - c[:, 0] * s[:, 1] * s[:, 2],
                        c[:, 0] * s[:, 1] * c[:, 2] + s[:, 0] * c[:, 1] * s[:, 2],
                        c[:, 0] * c[:, 1] * s[:, 2] - s[:, 0] * s[:, 1] * c[:, 2]], 1)
    size_xyz = torch.tensor([W, H, D], dtype=torch.float32)
    idx = torch.clamp((pos * (size_xyz - 1)).long(), min=0)
    inten = (vol[idx[:, 2], idx[:, 1], idx[:, 0]] / 10).unsqueeze(-1).contiguous()
    work = Workload(cfg, pos.contiguous(), scale, quat.contiguous(), inten,
                    {"kind": "spheres"}, seed)
    return work, vol


# The reference's multi-channel test (test/test_multi_channel.py:15-26): the
# same (100, 150, 80) volume in a (1.0, 1.5, 0.8) world (z, y, x) centred at
# (0.5, 0.7, 0.5), 5,000 Gaussians from random_gauss_init(anisotropicScale=True)
# without rotation, and two channels, the phantom's value and half of it.
REFERENCE_MULTICHANNEL = Config("ref_multichannel_test_100x150x80_5k_c2", (100, 150, 80), 5_000,
                                2, ("fixed", 0.03, 0.01, 0.02), "identity", (0.1, 1.0),
                                "uniform", "spheres", world=(1.0, 1.5, 0.8),
                                center=(0.5, 0.7, 0.5))


def reference_multichannel_scenario(seed: int = 0):
    """(Workload, phantom (D, H, W)) of the reference's multi-channel test, seeded.

    Positions U[0,1)^3 (world units, x y z); scales (0.02 * 1.5, 0.02 * 0.5,
    0.02) world units; identity rotations; channel 0 = the phantom's value at
    the voxel floor(pos * (size - 1)) per axis (random_gauss_init, not divided
    by 10 here), channel 1 = half of it (test_multi_channel.py:25)."""
    cfg = REFERENCE_MULTICHANNEL
    n = cfg.n
    D, H, W = cfg.vol
    vol = sphere_phantom(cfg.vol, np.random.default_rng(seed))
    g = torch.Generator(device="cpu").manual_seed(seed)
    pos = torch.rand((n, 3), generator=g, dtype=torch.float32)
    scale = torch.tensor([0.03, 0.01, 0.02], dtype=torch.float32).expand(n, 3).contiguous()
    quat = torch.zeros((n, 4), dtype=torch.float32)
    quat[:, 0] = 1.0
    size_xyz = torch.tensor([W, H, D], dtype=torch.float32)
    idx = torch.clamp((pos * (size_xyz - 1)).long(), min=0)
    one = vol[idx[:, 2], idx[:, 1], idx[:, 0]].unsqueeze(-1)
    inten = torch.cat([one, one / 2], dim=1).contiguous()
    work = Workload(cfg, pos.contiguous(), scale, quat, inten, {"kind": "spheres"}, seed)
    return work, vol


def volume_scaling_scenario(edge: int, seed: int = 0, base_edge: int = 96,
                            base_gaussians: int = 6000) -> Workload:
    """The reference's volume-scaling case (test/test_volume_scaling.py:53-64,
    130-139), seeded: a cubic volume of `edge` voxels in a unit world centred
    at 0.5, round(base_gaussians * edge / base_edge) Gaussians from
    random_gauss_init(anisotropicScale=True) (test/utils.py:91-154): positions
    U[0,1)^3, scales (0.03, 0.01, 0.02) world units, identity rotations, and
    intensities read from generate_noise_volume (test/utils.py:32-71:
    0.1 + 0.9 * avg_pool3d_5(U[0,1)), clamped to [0, 1]) at the voxel
    floor(pos * (edge - 1)).  The smoothed noise is not formed over the whole
    volume (6.9 GB at 1200^3): each Gaussian's value is 0.1 + 0.9 times the
    mean of 125 uniform draws of its own, the same distribution at an interior
    voxel (nearby Gaussians do not share draws, which nothing here depends on)."""
    n = max(1, int(round(base_gaussians * edge / base_edge)))
    cfg = Config(f"volume_scaling_{edge}cube_{n // 1000}k", (edge, edge, edge), n, 1,
                 ("fixed", 0.03, 0.01, 0.02), "identity", (0.1, 1.0), "uniform", "noise")
    g = torch.Generator(device="cpu").manual_seed(seed)
    pos = torch.rand((n, 3), generator=g, dtype=torch.float32)
    scale = torch.tensor([0.03, 0.01, 0.02], dtype=torch.float32).expand(n, 3).contiguous()
    quat = torch.zeros((n, 4), dtype=torch.float32)
    quat[:, 0] = 1.0
    u = torch.rand((n, 125), generator=g, dtype=torch.float32).mean(1, keepdim=True)
    inten = (0.1 + 0.9 * u).clamp(0.0, 1.0).contiguous()
    return Workload(cfg, pos.contiguous(), scale, quat, inten, {"kind": "noise"}, seed)
