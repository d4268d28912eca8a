"""Binning of Gaussians into 8x8x8 voxel tiles.

Drop-in for gs_voxelizer/bin_and_sort_gaussians.py of the reference (lines
14-54): same function, arguments and outputs.  The key duplication, stable
radix sort and tile-range extraction run in libgsvox.so.
"""
from typing import Tuple

from torch import Tensor

import gs_voxelizer.cuda as _C


def bin_and_sort_gaussians(
    num_gaussians: int,
    num_intersects: int,
    tile_min: Tensor,
    tile_max: Tensor,
    cum_tiles_hit: Tensor,
    vol_size: Tuple[int, int, int],
) -> Tuple[Tensor, Tensor]:
    """Map Gaussians to (tile, gaussian) intersections sorted by tile.

    Not differentiable.

    Args:
        num_gaussians: number of Gaussians N.
        num_intersects: total number of (tile, Gaussian) intersections,
            cum_tiles_hit[-1].
        tile_min, tile_max: (N, 3) int32 [min, max) tile boxes (x, y, z).
        cum_tiles_hit: (N,) int32 inclusive prefix sum of the per-Gaussian
            tile counts.
        vol_size: (D, H, W) = (z, y, x) voxel counts.

    Returns:
        gaussian_ids_sorted: (num_intersects,) int32 Gaussian ids ordered by
            tile id, ascending Gaussian id within a tile.
        tile_bins: (T, 2) int32 [start, end) ranges into gaussian_ids_sorted
            per tile (zeros for empty tiles), T = ceil(W/8)*ceil(H/8)*ceil(D/8).
    """
    gaussian_ids_sorted, tile_bins = _C.bin_and_sort_gaussians(
        num_gaussians,
        num_intersects,
        tile_min.contiguous(),
        tile_max.contiguous(),
        cum_tiles_hit.contiguous(),
        vol_size,
    )
    return gaussian_ids_sorted.contiguous(), tile_bins.contiguous()
