#!/usr/bin/env python3
"""Writes the golden fixtures of this directory from the CPU oracle.

The reference ships no golden data for this path (its only value test compares
live against an external CUDA package), so these fixtures freeze the oracle's
outputs on small seeded scenes: a regression pin for the oracle itself
(test_golden.py) and a stored target for the HIP path (test_gpu_golden.py).
Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "gs-voxelizer_amd")]

import oracle as O  # noqa: E402
from gs_voxelizer import synthetic as S  # noqa: E402

SCENES = {
    # README-style scene (cfg1 distributions) on a small volume with edge tiles
    "readme_small": S.Config("readme_small", (20, 24, 17), 300, 1, ("axis", 0.5, 4.0), "random",
                             (0.0, 1.0), "uniform", "smooth"),
    # the reference's multi-channel scenario: non-cubic world, off-centre volume
    "multichannel_c3": S.Config("multichannel_c3", (16, 30, 22), 200, 3, ("axis", 0.5, 3.0),
                                "random", (0.0, 1.0), "uniform", "smooth",
                                world=(1.0, 1.5, 0.8), center=(0.5, 0.7, 0.5)),
}


def make(name, cfg, seed=0):
    w = S.make_gaussians(cfg, seed=seed)
    p, s, q, I = (t.numpy() for t in (w.pos3d, w.scale3d, w.quat, w.intensities))
    g = np.random.default_rng(seed + 100).standard_normal(cfg.vol + (cfg.channels,)).astype(np.float32)
    r = O.pipeline(p, s, q, I, cfg.vol, cfg.world, cfg.center, vol_grad=g)
    _, amb_vol = O.voxelize_fwd(cfg.vol, r["gaussian_ids_sorted"], r["tile_bins"],
                                r["pos3d_radii"], r["conics"], I, with_amb=True)
    _, absum, amb = O.voxelize_bwd(cfg.vol, r["gaussian_ids_sorted"], r["tile_bins"],
                                   r["pos3d_radii"], r["conics"], I, g, diagnostics=True)
    out = dict(vol_size=np.array(cfg.vol), world=np.array(cfg.world), center=np.array(cfg.center),
               pos3d=p, scale3d=s, quat=q, intensities=I, vol_grad=g,
               amb_volume=amb_vol, abs_dpos3d_radii=absum[0], abs_dconics=absum[1],
               abs_dintensities=absum[2], amb_dpos3d_radii=amb[0], amb_dconics=amb[1],
               amb_dintensities=amb[2])
    for k in ("pos3d_radii", "conics", "tile_min", "tile_max", "num_tiles_hit", "cum_tiles_hit",
              "gaussian_ids_sorted", "tile_bins", "volume", "dpos3d_radii", "dconics",
              "dintensities", "dpos3d", "dscale3d", "dquat"):
        out[k] = r[k]
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes;", r["num_intersects"], "intersections")


if __name__ == "__main__":
    for name, cfg in SCENES.items():
        make(name, cfg)
