"""Projection: optimisation parameters -> rendering parameters, with autograd.

Drop-in for gs_voxelizer/optim_to_render.py of the reference (same function,
arguments, validation and return values, lines 12-149); the arithmetic runs in
the gfx950 kernels of libgsvox.so via ``gs_voxelizer.cuda``.
"""
from typing import Optional, Tuple

from torch import Tensor
from torch.autograd import Function

import gs_voxelizer.cuda as _C


def optim_to_render(
    pos3d: Tensor,
    scale3d: Tensor,
    quat: Tensor,
    intensities: Tensor,
    vol_size_voxel: Tuple[int, int, int],
    vol_size_world: Tuple[float, float, float],
    vol_center_pos: Tuple[float, float, float],
    pos3d_radii_buffer: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Convert Gaussians from optimisation-oriented to rendering-oriented parameters.

    Args:
        pos3d: (N, 3) Gaussian centres in world units (x, y, z).
        scale3d: (N, 3) per-axis scales in world units.
        quat: (N, 4) rotations as [w, x, y, z] (normalised internally).
        intensities: (N, C) intensities, 1 <= C <= 4.
        vol_size_voxel: (D, H, W) = (z, y, x) voxel counts.
        vol_size_world: world extent of the volume, (z, y, x).
        vol_center_pos: world position of the volume centre, (z, y, x).
        pos3d_radii_buffer: optional preallocated contiguous (N, 4) tensor, same
            dtype and device, that receives the returned positions/radii.

    Returns:
        pos3d_radii (N, 4): voxel-space centre (x, y, z) and radius in w,
        conics (N, 6): inverse voxel-space covariance (00, 01, 02, 11, 12, 22),
        tile_min (N, 3), tile_max (N, 3): int32 [min, max) tile box (x, y, z),
        num_tiles_hit (N,): int32 number of tiles in the box.
    The int32 outputs carry no gradient; intensities get no gradient from here.
    """
    return _OptimToRender.apply(
        pos3d.contiguous(),
        scale3d.contiguous(),
        quat.contiguous(),
        intensities.contiguous(),
        vol_size_voxel,
        vol_size_world,
        vol_center_pos,
        pos3d_radii_buffer,
    )


class _OptimToRender(Function):
    @staticmethod
    def forward(ctx, pos3d, scale3d, quat, intensities, vol_size_voxel, vol_size_world,
                vol_center_pos, pos3d_radii_buffer):
        num_gaussians = pos3d.size(-2)
        if num_gaussians < 1 or pos3d.shape[-1] != 3:
            raise ValueError(f"Invalid shape for pos3d: {pos3d.shape}")
        pos3d_radii, conics, tile_min, tile_max, num_tiles_hit = _C.optim_to_render_forward(
            num_gaussians, pos3d, scale3d, quat, intensities, vol_size_voxel, vol_size_world,
            vol_center_pos)
        ctx.num_gaussians = num_gaussians
        ctx.vol_size_voxel = vol_size_voxel
        ctx.vol_size_world = vol_size_world
        ctx.vol_center_pos = vol_center_pos
        ctx.save_for_backward(pos3d, scale3d, quat, pos3d_radii)
        ctx.mark_non_differentiable(tile_min, tile_max, num_tiles_hit)
        # gradients of unused outputs arrive as None (handled in backward) rather
        # than as zero tensors the engine would fill, one launch each
        ctx.set_materialize_grads(False)
        if pos3d_radii_buffer is not None:
            buf = pos3d_radii_buffer
            if not buf.is_contiguous():
                raise ValueError("pos3d_radii_buffer must be contiguous")
            if buf.shape != pos3d_radii.shape:
                raise ValueError(
                    f"pos3d_radii_buffer shape mismatch: expected {pos3d_radii.shape}, "
                    f"got {buf.shape}")
            if buf.device != pos3d_radii.device:
                raise ValueError("pos3d_radii_buffer must be on the same device as inputs")
            if buf.dtype != pos3d_radii.dtype:
                raise ValueError("pos3d_radii_buffer must share dtype with inputs")
            buf.copy_(pos3d_radii)
            returned = buf
        else:
            returned = pos3d_radii
        return returned, conics, tile_min, tile_max, num_tiles_hit

    @staticmethod
    def backward(ctx, pos3d_radii_grad, conics_grad, _tile_min_grad, _tile_max_grad,
                 _num_tiles_grad):
        pos3d, scale3d, quat, pos3d_radii = ctx.saved_tensors
        if pos3d_radii_grad is None:
            pos3d_radii_grad = pos3d_radii.new_zeros(pos3d_radii.shape)
        if conics_grad is None:
            conics_grad = pos3d_radii.new_zeros((pos3d_radii.shape[0], 6))
        grad_pos3d, grad_scale3d, grad_quat = _C.optim_to_render_backward(
            ctx.num_gaussians, pos3d, scale3d, quat, ctx.vol_size_voxel, ctx.vol_size_world,
            ctx.vol_center_pos, pos3d_radii_grad, conics_grad, pos3d_radii)
        return grad_pos3d, grad_scale3d, grad_quat, None, None, None, None, None
