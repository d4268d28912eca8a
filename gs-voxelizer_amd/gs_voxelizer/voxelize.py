"""Differentiable voxelization of projected Gaussians into a (D, H, W, C) grid.

Drop-in for gs_voxelizer/voxelize.py of the reference (lines 14-173): same
function, arguments, empty-input behaviour and autograd outputs.  The prefix sum
of tile counts, binning, forward and backward run in libgsvox.so.

The reference reads the intersection count back to the host before binning
(voxelize.py:87-88), which idles the GPU for a round trip every forward.  Here
the first forward on a device does the same and records a capacity; later
forwards launch binning and the forward kernel at that capacity with the count
left on the device, copy the count to pinned host memory meanwhile, and check
it after the launches.  A count above the capacity (the scene grew) reruns
binning and the forward with the exact count and raises the capacity; results
are identical either way.  GSV_SYNC_COUNT=1 restores the reference's host read.
"""
import os
from typing import Tuple

import torch
from torch import Tensor
from torch.autograd import Function

import gs_voxelizer.cuda as _C

from .bin_and_sort_gaussians import bin_and_sort_gaussians

_INT32_MAX = 2**31 - 1
_capacity = {}  # device index -> intersection capacity of the speculative path


def _grow(count: int) -> int:
    return min(_INT32_MAX, count + count // 4 + 4096)


def _speculate() -> bool:
    return os.environ.get("GSV_SYNC_COUNT", "0") != "1"


def voxelize_gaussians(
    pos3d_radii: Tensor,
    conics: Tensor,
    intensities: Tensor,
    vol_size_voxel: Tuple[int, int, int],
    tile_min: Tensor,
    tile_max: Tensor,
    num_tiles_hit: Tensor,
    use_per_gaussian_backward: bool = True,
) -> Tensor:
    """Voxelize 3D Gaussians into a voxel grid.

    Args:
        pos3d_radii: (N, 4) voxel-space centres (x, y, z), radius in w.
        conics: (N, 6) inverse covariances (from optim_to_render).
        intensities: (N, C) intensities, C <= 4 (a 1-D tensor is treated as C=1).
        vol_size_voxel: (D, H, W) = (z, y, x) output size.
        tile_min, tile_max, num_tiles_hit: tile boxes and counts from optim_to_render.
        use_per_gaussian_backward: selects the reference's per-Gaussian (True) or
            per-voxel (False) backward kernel; both produce the same gradients
            here (one kernel serves both).

    Returns:
        (D, H, W, C) float32 volume.
    """
    return _VoxelizeGaussians.apply(
        pos3d_radii.contiguous(),
        conics.contiguous(),
        intensities.contiguous(),
        vol_size_voxel,
        tile_min,
        tile_max,
        num_tiles_hit,
        use_per_gaussian_backward,
    )


class _VoxelizeGaussians(Function):
    @staticmethod
    def forward(ctx, pos3d_radii, conics, intensities, vol_size_voxel, tile_min, tile_max,
                num_tiles_hit, use_per_gaussian_backward=False):
        if intensities.dim() == 1:
            intensities = intensities.unsqueeze(-1)
        num_gaussians = pos3d_radii.size(-2)
        ctx.vol_size_voxel = vol_size_voxel
        ctx.use_per_gaussian_backward = use_per_gaussian_backward
        dev = pos3d_radii.device
        D, H, W = (int(v) for v in vol_size_voxel)
        boxes = ()
        if num_gaussians == 0:
            out = torch.zeros(D, H, W, intensities.shape[-1], device=dev, dtype=pos3d_radii.dtype)
            gaussian_ids_sorted = torch.zeros(0, 1, device=dev, dtype=torch.int32)
            tile_bins = torch.zeros(0, 3, device=dev, dtype=torch.int32)
            ctx.num_intersects = 0
        else:
            cum_tiles_hit, total = _C.cumsum_tiles_hit(num_tiles_hit.contiguous())
            key = dev.index if dev.index is not None else torch.cuda.current_device()
            cap = _capacity.get(key) if _speculate() else None
            gaussian_ids_sorted = None
            if cap is not None:
                # launch at the recorded capacity; the count travels meanwhile
                host = torch.empty((1,), dtype=torch.int64, pin_memory=True)
                host.copy_(total, non_blocking=True)
                copied = torch.cuda.Event()
                copied.record()
                ids_cap, tile_bins = _C.bin_and_sort_gaussians_device_count(
                    num_gaussians, cap, total, tile_min, tile_max, cum_tiles_hit, vol_size_voxel)
                out = _C.voxelize_forward(vol_size_voxel, ids_cap, tile_bins, pos3d_radii, conics,
                                          intensities)
                copied.synchronize()  # the queued kernels keep the GPU busy meanwhile
                num_intersects = int(host[0])
                if num_intersects <= cap:
                    gaussian_ids_sorted = ids_cap[:num_intersects]
                    if num_intersects < cap // 4:
                        _capacity[key] = _grow(num_intersects)
            else:
                num_intersects = int(total.item())
            if num_intersects > _INT32_MAX:
                raise RuntimeError(
                    f"gs_voxelizer: {num_intersects} tile intersections overflow the int32 layout")
            ctx.num_intersects = num_intersects
            if num_intersects < 1:
                out = torch.zeros(D, H, W, intensities.shape[-1], device=dev)
                gaussian_ids_sorted = torch.zeros(0, 1, device=dev, dtype=torch.int32)
                tile_bins = torch.zeros(0, 3, device=dev, dtype=torch.int32)
            else:
                if gaussian_ids_sorted is None:  # first call, host read requested, or overflow
                    gaussian_ids_sorted, tile_bins = bin_and_sort_gaussians(
                        num_gaussians, num_intersects, tile_min, tile_max, cum_tiles_hit,
                        vol_size_voxel)
                    out = _C.voxelize_forward(vol_size_voxel, gaussian_ids_sorted, tile_bins,
                                              pos3d_radii, conics, intensities)
                    if _speculate():
                        _capacity[key] = _grow(num_intersects)
                # the backward reduces per-pair partials in duplication order (no atomics)
                boxes = (tile_min.contiguous(), tile_max.contiguous(), cum_tiles_hit)
        ctx.n_boxes = len(boxes)
        ctx.set_materialize_grads(False)  # an unused volume needs no zero-filled gradient
        ctx.save_for_backward(pos3d_radii, conics, intensities, gaussian_ids_sorted, tile_bins,
                              *boxes)
        return out

    @staticmethod
    def backward(ctx, vol_grad):
        vol_size_voxel = ctx.vol_size_voxel
        saved = ctx.saved_tensors
        pos3d_radii, conics, intensities, gaussian_ids_sorted, tile_bins = saved[:5]
        boxes = saved[5:]
        if ctx.num_intersects < 1 or vol_grad is None:
            pos3d_grad = torch.zeros_like(pos3d_radii)
            conics_grad = torch.zeros_like(conics)
            intensities_grad = torch.zeros_like(intensities)
        else:
            fn = (_C.voxelize_backward_per_gaussian if ctx.use_per_gaussian_backward
                  else _C.voxelize_backward)
            pos3d_grad, conics_grad, intensities_grad = fn(
                vol_size_voxel, gaussian_ids_sorted, tile_bins, pos3d_radii, conics, intensities,
                vol_grad.contiguous(), *boxes)
        return pos3d_grad, conics_grad, intensities_grad, None, None, None, None, None
