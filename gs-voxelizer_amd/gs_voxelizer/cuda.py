"""Native entry points of gs_voxelizer, backed by libgsvox.so (gfx950 HIP kernels).

Same module path, function names, argument order and return values as the
reference's pybind11 extension ``gs_voxelizer.cuda`` (gs_voxelizer/cuda/ext.cpp:4-11,
bindings.h:40-194), so ``import gs_voxelizer.cuda as _C`` callers keep working.
Outputs and workspaces are torch tensors allocated on the inputs' device; every
kernel is enqueued on torch's current stream of that device.  Errors raise
RuntimeError, as the reference's TORCH_CHECK / std::runtime_error do.

``cumsum_tiles_hit`` is an addition: the reference computes that prefix sum with
``torch.cumsum`` in voxelize.py:87; here it is a native kernel as well.
"""
import ctypes
from typing import Tuple

import torch

from . import _lib

MAX_CHANNELS = 4
BLOCK = 8

_L = _lib.load()


def _status_error(name: str, status: int) -> RuntimeError:
    text = _L.gsv_status_string(status).decode()
    if status == 5:  # GSV_ERR_HIP
        text += f" (hipError_t {_L.gsv_last_hip_error()})"
    return RuntimeError(f"gs_voxelizer.{name}: {text}")


def _call(name: str, *args) -> None:
    st = getattr(_L, "gsv_" + name)(*args)
    if st != 0:
        raise _status_error(name, st)


def _check_input(t: torch.Tensor, what: str) -> None:
    # CHECK_INPUT of bindings.h:7-12
    if not t.is_cuda:
        raise RuntimeError(f"{what} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{what} must be contiguous")


def _check_dtype(t: torch.Tensor, what: str, dtype: torch.dtype) -> None:
    if t.dtype != dtype:
        raise RuntimeError(f"{what}: expected scalar type {dtype} but found {t.dtype}")


def _check_rows(n: int, tensors) -> None:
    """The kernels index rows [0, num_points) of every per-Gaussian input: a
    count beyond a tensor's rows would read past its memory, so it is refused
    here (the reference's bindings take num_points as given)."""
    if n < 0:
        raise RuntimeError(f"num_points must be non-negative, got {n}")
    for t, w, width in tensors:
        if t.numel() < n * width:
            raise RuntimeError(f"{w} holds {t.numel() // max(width, 1)} rows, fewer than "
                               f"num_points = {n}")


def _ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr()) if t.numel() > 0 else ctypes.c_void_p(0)


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _tiles(vol_size) -> Tuple[int, int, int]:
    D, H, W = (int(v) for v in vol_size)
    return (W + BLOCK - 1) // BLOCK, (H + BLOCK - 1) // BLOCK, (D + BLOCK - 1) // BLOCK


def _channels(intensities: torch.Tensor) -> int:
    channels = intensities.size(1)  # 2-D required, bindings.cu:59
    if channels > MAX_CHANNELS:
        raise RuntimeError("Number of channels exceeds MAX_CHANNELS")
    return channels


def optim_to_render_forward(num_gaussians: int, pos3d, scale3d, quat, intensities,
                            vol_size_voxel, vol_size_world, vol_center_pos):
    """bindings.cu:38-189. Returns (pos3d_radii, conics, tile_min, tile_max, num_tiles_hit)."""
    for t, w in ((pos3d, "pos3d"), (scale3d, "scale3d"), (quat, "quat"), (intensities, "intensities")):
        _check_input(t, w)
        _check_dtype(t, w, torch.float32)
    channels = _channels(intensities)
    n = int(num_gaussians)
    _check_rows(n, ((pos3d, "pos3d", 3), (scale3d, "scale3d", 3), (quat, "quat", 4),
                    (intensities, "intensities", channels)))
    D, H, W = (int(v) for v in vol_size_voxel)
    wz, wy, wx = (float(v) for v in vol_size_world)
    cz, cy, cx = (float(v) for v in vol_center_pos)
    dev = pos3d.device
    f32 = dict(device=dev, dtype=torch.float32)
    i32 = dict(device=dev, dtype=torch.int32)
    pos3d_radii = torch.empty((n, 4), **f32)
    conics = torch.empty((n, 6), **f32)
    tile_min = torch.empty((n, 3), **i32)
    tile_max = torch.empty((n, 3), **i32)
    num_tiles_hit = torch.empty((n,), **i32)
    with torch.cuda.device(dev):
        _call("project_fwd", n, channels, _ptr(pos3d), _ptr(scale3d), _ptr(quat), _ptr(intensities),
              D, H, W, wz, wy, wx, cz, cy, cx, _ptr(pos3d_radii), _ptr(conics), _ptr(tile_min),
              _ptr(tile_max), _ptr(num_tiles_hit), _stream(dev))
    return pos3d_radii, conics, tile_min, tile_max, num_tiles_hit


def optim_to_render_backward(num_gaussians: int, pos3d, scale3d, quat, vol_size_voxel,
                             vol_size_world, vol_center_pos, pos3d_radii_grad_in, conics_grad_in,
                             pos3d_radii_out):
    """bindings.cu:197-251. Returns (grad_pos3d, grad_scale3d, grad_quat)."""
    n = int(num_gaussians)
    dev = pos3d.device
    scale3d, quat = scale3d.contiguous(), quat.contiguous()
    dpr = pos3d_radii_grad_in.contiguous()
    dcn = conics_grad_in.contiguous()
    pr = pos3d_radii_out.contiguous()
    for t, w in ((scale3d, "scale3d"), (quat, "quat"), (dpr, "pos3d_radii_grad_in"),
                 (dcn, "conics_grad_in"), (pr, "pos3d_radii_out")):
        _check_input(t, w)
        _check_dtype(t, w, torch.float32)
    _check_rows(n, ((pos3d, "pos3d", 3), (scale3d, "scale3d", 3), (quat, "quat", 4),
                    (dpr, "pos3d_radii_grad_in", 4), (dcn, "conics_grad_in", 6),
                    (pr, "pos3d_radii_out", 4)))
    D, H, W = (int(v) for v in vol_size_voxel)
    wz, wy, wx = (float(v) for v in vol_size_world)
    cz, cy, cx = (float(v) for v in vol_center_pos)
    f32 = dict(device=dev, dtype=torch.float32)
    dpos = torch.empty((n, 3), **f32)
    dscale = torch.empty((n, 3), **f32)
    dquat = torch.empty((n, 4), **f32)
    with torch.cuda.device(dev):
        _call("project_bwd", n, _ptr(pos3d), _ptr(scale3d), _ptr(quat), D, H, W, wz, wy, wx,
              cz, cy, cx, _ptr(dpr), _ptr(dcn), _ptr(pr), _ptr(dpos), _ptr(dscale), _ptr(dquat),
              _stream(dev))
    return dpos, dscale, dquat


def cumsum_tiles_hit(num_tiles_hit, total_host=None):
    """Inclusive int32 prefix sum of num_tiles_hit plus its total as a (1,) int64
    device tensor (one scalar to read back instead of the whole array).

    total_host: optional (1,) int64 pinned CPU tensor (pin_memory=True) that the
    scan kernel writes the total into as well; it holds the count once an event
    recorded after this call has completed, without a device-to-host copy."""
    _check_input(num_tiles_hit, "num_tiles_hit")
    _check_dtype(num_tiles_hit, "num_tiles_hit", torch.int32)
    if total_host is not None:
        if (total_host.is_cuda or not total_host.is_pinned() or total_host.dtype != torch.int64
                or total_host.numel() != 1):
            raise RuntimeError("total_host must be a pinned (1,) int64 CPU tensor")
    n = num_tiles_hit.numel()
    dev = num_tiles_hit.device
    cum = torch.empty((n,), device=dev, dtype=torch.int32)
    total = torch.empty((1,), device=dev, dtype=torch.int64)  # written by the scan
    nbytes = ctypes.c_size_t(0)
    _call("scan_workspace_bytes", n, ctypes.byref(nbytes))
    ws = torch.empty((max(nbytes.value, 1),), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _call("cumsum_tiles_hit", n, _ptr(num_tiles_hit), _ptr(cum), _ptr(total),
              _ptr(total_host) if total_host is not None else ctypes.c_void_p(0), _ptr(ws),
              nbytes.value, _stream(dev))
    return cum, total


def bin_and_sort_gaussians(num_gaussians: int, num_intersects: int, tile_min, tile_max,
                           cum_tiles_hit, vol_size, return_tiles: bool = False):
    """bindings.cu:259-360. Returns (gaussian_ids_sorted (I,), tile_bins (T,2)), plus
    the tile id of each sorted pair (I,) when return_tiles (the sort's keys, which
    voxelize_backward* take as tiles_sorted)."""
    for t, w in ((tile_min, "tile_min"), (tile_max, "tile_max"), (cum_tiles_hit, "cum_tiles_hit")):
        _check_input(t, w)
        _check_dtype(t, w, torch.int32)
    Tx, Ty, Tz = _tiles(vol_size)
    T = Tx * Ty * Tz
    D, H, W = (int(v) for v in vol_size)
    dev = tile_min.device
    n, I = int(num_gaussians), int(num_intersects)
    _check_rows(n, ((tile_min, "tile_min", 3), (tile_max, "tile_max", 3),
                    (cum_tiles_hit, "cum_tiles_hit", 1)))
    i32 = dict(device=dev, dtype=torch.int32)
    tile_bins = torch.empty((T, 2), **i32)
    ids = torch.empty((max(I, 0),), **i32)
    tiles = torch.empty((max(I, 0),), **i32) if return_tiles else None
    nbytes = ctypes.c_size_t(0)
    _call("bin_workspace_bytes", n, max(I, 0), D, H, W, ctypes.byref(nbytes))
    ws = torch.empty((max(nbytes.value, 1),), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _call("bin_and_sort", n, I, _ptr(tile_min), _ptr(tile_max), _ptr(cum_tiles_hit), D, H, W,
              _ptr(ws), nbytes.value, _ptr(ids), _ptr(tile_bins),
              _ptr(tiles) if tiles is not None else ctypes.c_void_p(0), _stream(dev))
    return (ids, tile_bins, tiles) if return_tiles else (ids, tile_bins)


def bin_and_sort_gaussians_device_count(num_gaussians: int, capacity: int, num_intersects_dev,
                                        tile_min, tile_max, cum_tiles_hit, vol_size,
                                        return_tiles: bool = False):
    """Binning without the host read of the pair count (voxelize.py:87-88).

    num_intersects_dev is a (1,) int64 device tensor, e.g. the total returned by
    cumsum_tiles_hit.  Returns (gaussian_ids_sorted (capacity,), tile_bins (T,2)):
    the first min(count, capacity) ids are sorted, and the result is complete only
    when count <= capacity, which the caller checks once the count is on the host.
    With return_tiles the tile id of each sorted pair (capacity,) follows.
    """
    for t, w in ((tile_min, "tile_min"), (tile_max, "tile_max"), (cum_tiles_hit, "cum_tiles_hit"),
                 (num_intersects_dev, "num_intersects_dev")):
        _check_input(t, w)
    for t, w in ((tile_min, "tile_min"), (tile_max, "tile_max"), (cum_tiles_hit, "cum_tiles_hit")):
        _check_dtype(t, w, torch.int32)
    _check_dtype(num_intersects_dev, "num_intersects_dev", torch.int64)
    Tx, Ty, Tz = _tiles(vol_size)
    D, H, W = (int(v) for v in vol_size)
    dev = tile_min.device
    n, cap = int(num_gaussians), max(int(capacity), 0)
    _check_rows(n, ((tile_min, "tile_min", 3), (tile_max, "tile_max", 3),
                    (cum_tiles_hit, "cum_tiles_hit", 1)))
    i32 = dict(device=dev, dtype=torch.int32)
    tile_bins = torch.empty((Tx * Ty * Tz, 2), **i32)
    ids = torch.empty((cap,), **i32)
    tiles = torch.empty((cap,), **i32) if return_tiles else None
    nbytes = ctypes.c_size_t(0)
    _call("bin_workspace_bytes", n, cap, D, H, W, ctypes.byref(nbytes))
    ws = torch.empty((max(nbytes.value, 1),), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _call("bin_and_sort_device_count", n, cap, _ptr(num_intersects_dev), _ptr(tile_min),
              _ptr(tile_max), _ptr(cum_tiles_hit), D, H, W, _ptr(ws), nbytes.value, _ptr(ids),
              _ptr(tile_bins), _ptr(tiles) if tiles is not None else ctypes.c_void_p(0),
              _stream(dev))
    return (ids, tile_bins, tiles) if return_tiles else (ids, tile_bins)


def cumsum_bin_and_sort_device_count(num_gaussians: int, capacity: int, num_tiles_hit, tile_min,
                                     tile_max, vol_size, total_host=None,
                                     return_tiles: bool = False):
    """cumsum_tiles_hit followed by bin_and_sort_gaussians_device_count, in
    one native call (voxelize.py:87-88 and the binning, without the host read
    of the count).  Returns (cum_tiles_hit, total, gaussian_ids_sorted
    (capacity,), tile_bins (T,2)) and, with return_tiles, the tile of each
    sorted pair (capacity,); total_host as for cumsum_tiles_hit.  The binning
    is complete only when total <= capacity, which the caller checks."""
    for t, w in ((num_tiles_hit, "num_tiles_hit"), (tile_min, "tile_min"),
                 (tile_max, "tile_max")):
        _check_input(t, w)
        _check_dtype(t, w, torch.int32)
    if total_host is not None:
        if (total_host.is_cuda or not total_host.is_pinned() or total_host.dtype != torch.int64
                or total_host.numel() != 1):
            raise RuntimeError("total_host must be a pinned (1,) int64 CPU tensor")
    Tx, Ty, Tz = _tiles(vol_size)
    D, H, W = (int(v) for v in vol_size)
    dev = tile_min.device
    n, cap = int(num_gaussians), max(int(capacity), 0)
    _check_rows(n, ((tile_min, "tile_min", 3), (tile_max, "tile_max", 3),
                    (num_tiles_hit, "num_tiles_hit", 1)))
    i32 = dict(device=dev, dtype=torch.int32)
    cum = torch.empty((n,), **i32)
    total = torch.empty((1,), device=dev, dtype=torch.int64)
    tile_bins = torch.empty((Tx * Ty * Tz, 2), **i32)
    ids = torch.empty((cap,), **i32)
    tiles = torch.empty((cap,), **i32) if return_tiles else None
    nbytes = ctypes.c_size_t(0)
    _call("cumsum_bin_workspace_bytes", n, cap, D, H, W, ctypes.byref(nbytes))
    ws = torch.empty((max(nbytes.value, 1),), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _call("cumsum_bin_and_sort_device_count", n, cap, _ptr(num_tiles_hit), _ptr(tile_min),
              _ptr(tile_max), D, H, W, _ptr(cum), _ptr(total),
              _ptr(total_host) if total_host is not None else ctypes.c_void_p(0), _ptr(ws),
              nbytes.value, _ptr(ids), _ptr(tile_bins),
              _ptr(tiles) if tiles is not None else ctypes.c_void_p(0), _stream(dev))
    out = (cum, total, ids, tile_bins)
    return out + (tiles,) if return_tiles else out


def _voxelize_inputs(gaussian_ids_sorted, tile_bins, pos3d, conics, intensities):
    for t, w in ((gaussian_ids_sorted, "gaussian_ids_sorted"), (tile_bins, "tile_bins"),
                 (pos3d, "pos3d"), (conics, "conics"), (intensities, "intensities")):
        _check_input(t, w)
    _check_dtype(gaussian_ids_sorted, "gaussian_ids_sorted", torch.int32)
    _check_dtype(tile_bins, "tile_bins", torch.int32)
    for t, w in ((pos3d, "pos3d"), (conics, "conics"), (intensities, "intensities")):
        _check_dtype(t, w, torch.float32)


def _pair_flags(pair_live, n_pairs):
    """ctypes pointer of the optional per-pair cull flags (uint8, >= n_pairs)."""
    if pair_live is None:
        return ctypes.c_void_p(0)
    _check_input(pair_live, "pair_live")
    _check_dtype(pair_live, "pair_live", torch.uint8)
    if pair_live.numel() < n_pairs:
        raise RuntimeError("pair_live must hold one byte per sorted pair")
    return _ptr(pair_live)


def voxelize_forward(vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics, intensities,
                     pair_live=None):
    """bindings.cu:362-457. Returns the (D, H, W, C) volume.

    pair_live (optional, uint8, one per sorted pair) receives 1 for every pair
    the kernel evaluated and 0 for each it culled (no voxel centre of the tile
    inside the Gaussian's gate); handing it to the backward skips those pairs
    there too."""
    _voxelize_inputs(gaussian_ids_sorted, tile_bins, pos3d, conics, intensities)
    channels = _channels(intensities)
    D, H, W = (int(v) for v in vol_size)
    n = pos3d.size(0)
    dev = pos3d.device
    out = torch.empty((D, H, W, channels), device=dev, dtype=torch.float32)
    Tx, Ty, Tz = _tiles(vol_size)
    if tile_bins.numel() < 2 * Tx * Ty * Tz:
        raise RuntimeError("tile_bins does not cover the volume's tile grid")
    with torch.cuda.device(dev):
        _call("voxelize_fwd", D, H, W, channels, n, gaussian_ids_sorted.numel(),
              _ptr(gaussian_ids_sorted), _ptr(tile_bins), _ptr(pos3d), _ptr(conics),
              _ptr(intensities), _ptr(out), _pair_flags(pair_live, gaussian_ids_sorted.numel()),
              _stream(dev))
    return out


def _l1_target(target, volume):
    """The target laid out like the (D, H, W, C) volume (a (D, H, W) target serves C = 1)."""
    _check_input(target, "target")
    _check_dtype(target, "target", torch.float32)
    if target.device != volume.device:
        raise RuntimeError("target must be on the volume's device")
    if target.shape == volume.shape:
        return target
    if target.dim() == 3 and volume.shape[-1] == 1 and tuple(target.shape) == tuple(volume.shape[:3]):
        return target
    raise RuntimeError(f"target shape {tuple(target.shape)} does not match the volume "
                       f"{tuple(volume.shape)}")


def voxelize_forward_l1(vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics, intensities,
                        target, pair_live=None):
    """voxelize_forward fused with torch.nn.functional.l1_loss(volume, target) (mean).
    Returns (volume (D, H, W, C), loss (0-d device tensor), sign): sign is
    sgn(volume - target) as int8 (0 where the difference is NaN, as torch's sign), kept for
    voxelize_backward_l1.  pair_live as in voxelize_forward."""
    _voxelize_inputs(gaussian_ids_sorted, tile_bins, pos3d, conics, intensities)
    channels = _channels(intensities)
    D, H, W = (int(v) for v in vol_size)
    n = pos3d.size(0)
    dev = pos3d.device
    out = torch.empty((D, H, W, channels), device=dev, dtype=torch.float32)
    target = _l1_target(target, out)
    sign = torch.empty((D, H, W, channels), device=dev, dtype=torch.int8)
    loss = torch.empty((), device=dev, dtype=torch.float32)
    Tx, Ty, Tz = _tiles(vol_size)
    if tile_bins.numel() < 2 * Tx * Ty * Tz:
        raise RuntimeError("tile_bins does not cover the volume's tile grid")
    nbytes = ctypes.c_size_t(0)
    _call("voxelize_fwd_l1_workspace_bytes", D, H, W, ctypes.byref(nbytes))
    ws = torch.empty((max(nbytes.value, 1),), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _call("voxelize_fwd_l1", D, H, W, channels, n, gaussian_ids_sorted.numel(),
              _ptr(gaussian_ids_sorted), _ptr(tile_bins), _ptr(pos3d), _ptr(conics),
              _ptr(intensities), _ptr(target), _ptr(out), _ptr(sign), _ptr(loss),
              _pair_flags(pair_live, gaussian_ids_sorted.numel()), _ptr(ws), nbytes.value,
              _stream(dev))
    return out, loss, sign


def _voxelize_backward(variant, vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics,
                       intensities, vol_grad_in, tile_min=None, tile_max=None,
                       cum_tiles_hit=None, l1=None, tiles_sorted=None, count_dev=None,
                       pair_live=None):
    """l1 = (sign, grad_loss): the fused L1 source, with vol_grad_in optional.
    tiles_sorted: the binning's tile id per sorted pair (return_tiles), optional.
    count_dev: (1,) int64 device tensor with the live pair count, when the id
    arrays are capacity-sized (bin_and_sort_gaussians_device_count); optional.
    pair_live: the forward's cull flags (voxelize_forward(..., pair_live=)),
    optional; the backward then skips the culled pairs (same gradients)."""
    _voxelize_inputs(gaussian_ids_sorted, tile_bins, pos3d, conics, intensities)
    given = [t is not None for t in (tile_min, tile_max, cum_tiles_hit)]
    if any(given) and not all(given):
        raise RuntimeError("tile_min, tile_max and cum_tiles_hit must be given together")
    deterministic = all(given)
    if deterministic:
        for t, w in ((tile_min, "tile_min"), (tile_max, "tile_max"),
                     (cum_tiles_hit, "cum_tiles_hit")):
            _check_input(t, w)
            _check_dtype(t, w, torch.int32)
    channels = _channels(intensities)
    D, H, W = (int(v) for v in vol_size)
    if vol_grad_in is not None or l1 is None:
        _check_input(vol_grad_in, "vol_grad_in")
        _check_dtype(vol_grad_in, "vol_grad_in", torch.float32)
        if vol_grad_in.numel() != D * H * W * channels:
            raise RuntimeError("vol_grad_in must have D*H*W*channels elements")
    if l1 is not None:
        sign, grad_loss = l1
        _check_input(sign, "sign")
        _check_dtype(sign, "sign", torch.int8)
        _check_input(grad_loss, "grad_loss")
        _check_dtype(grad_loss, "grad_loss", torch.float32)
        if sign.numel() != D * H * W * channels or grad_loss.numel() != 1:
            raise RuntimeError("sign must have D*H*W*channels elements and grad_loss one")
    n = pos3d.size(0)
    dev = pos3d.device
    I = gaussian_ids_sorted.numel()
    if count_dev is not None:
        _check_input(count_dev, "count_dev")
        _check_dtype(count_dev, "count_dev", torch.int64)
    if tiles_sorted is not None:
        _check_input(tiles_sorted, "tiles_sorted")
        _check_dtype(tiles_sorted, "tiles_sorted", torch.int32)
        if tiles_sorted.numel() < I:
            raise RuntimeError("tiles_sorted must hold a tile id for every sorted pair")
    Tx, Ty, Tz = _tiles(vol_size)
    if I > 0 and tile_bins.numel() < 2 * Tx * Ty * Tz:
        raise RuntimeError("tile_bins does not cover the volume's tile grid")
    f32 = dict(device=dev, dtype=torch.float32)
    dpos = torch.empty((n, 4), **f32)
    dconics = torch.empty((n, 6), **f32)
    dint = torch.empty((n, channels), **f32)
    nbytes = ctypes.c_size_t(0)
    _call("voxelize_bwd_workspace_bytes", D, H, W, channels, n, I, int(deterministic),
          ctypes.byref(nbytes))
    ws = torch.empty((max(nbytes.value, 1),), device=dev, dtype=torch.uint8)
    null = ctypes.c_void_p(0)
    boxes = ((_ptr(tile_min), _ptr(tile_max), _ptr(cum_tiles_hit)) if deterministic
             else (null, null, null))
    vg = _ptr(vol_grad_in) if vol_grad_in is not None else null
    ts = _ptr(tiles_sorted) if tiles_sorted is not None else null
    cd = _ptr(count_dev) if count_dev is not None else null
    pl = _pair_flags(pair_live, I)
    with torch.cuda.device(dev):
        if l1 is None:
            _call("voxelize_bwd", D, H, W, channels, n, I, _ptr(gaussian_ids_sorted),
                  _ptr(tile_bins), _ptr(pos3d), _ptr(conics), _ptr(intensities), vg, *boxes, ts,
                  cd, pl, _ptr(dpos), _ptr(dconics), _ptr(dint), variant, _ptr(ws), nbytes.value,
                  _stream(dev))
        else:
            _call("voxelize_bwd_l1", D, H, W, channels, n, I, _ptr(gaussian_ids_sorted),
                  _ptr(tile_bins), _ptr(pos3d), _ptr(conics), _ptr(intensities), _ptr(sign),
                  _ptr(grad_loss), vg, *boxes, ts, cd, pl, _ptr(dpos), _ptr(dconics), _ptr(dint),
                  variant, _ptr(ws), nbytes.value, _stream(dev))
    return dpos, dconics, dint


def voxelize_backward_l1(vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics, intensities,
                         sign, grad_loss, vol_grad_in=None, tile_min=None, tile_max=None,
                         cum_tiles_hit=None, per_gaussian=True, tiles_sorted=None,
                         count_dev=None, pair_live=None):
    """Backward of voxelize_forward_l1: dL/dvolume = sign * grad_loss / numel (+
    vol_grad_in, the volume's gradient from other uses, when given), never
    materialised.  Returns (dpos3d_radii, dconics, dintensities)."""
    return _voxelize_backward(1 if per_gaussian else 0, vol_size, gaussian_ids_sorted, tile_bins,
                              pos3d, conics, intensities, vol_grad_in, tile_min, tile_max,
                              cum_tiles_hit, l1=(sign, grad_loss), tiles_sorted=tiles_sorted,
                              count_dev=count_dev, pair_live=pair_live)


def voxelize_backward(vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics, intensities,
                      vol_grad_in, tile_min=None, tile_max=None, cum_tiles_hit=None,
                      tiles_sorted=None, count_dev=None, pair_live=None):
    """bindings.cu:459-584 (per-voxel variant). Returns (dpos3d_radii, dconics, dintensities).

    The optional tile_min / tile_max / cum_tiles_hit (the projection's tile boxes
    and the prefix sum used for binning) select the atomic-free, bitwise
    reproducible reduction; without them float atomics are used, as in the
    reference.  tiles_sorted (bin_and_sort_gaussians(..., return_tiles=True)) saves
    rebuilding the tile of each pair; count_dev gives the live pair count for
    capacity-sized id arrays; pair_live (the forward's cull flags) skips the pairs
    the forward culled."""
    return _voxelize_backward(0, vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics,
                              intensities, vol_grad_in, tile_min, tile_max, cum_tiles_hit,
                              tiles_sorted=tiles_sorted, count_dev=count_dev,
                              pair_live=pair_live)


def voxelize_backward_per_gaussian(vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics,
                                   intensities, vol_grad_in, tile_min=None, tile_max=None,
                                   cum_tiles_hit=None, tiles_sorted=None, count_dev=None,
                                   pair_live=None):
    """bindings.cu:586-781 (per-Gaussian variant). Returns (dpos3d_radii, dconics, dintensities).
    Optional arguments as in voxelize_backward."""
    return _voxelize_backward(1, vol_size, gaussian_ids_sorted, tile_bins, pos3d, conics,
                              intensities, vol_grad_in, tile_min, tile_max, cum_tiles_hit,
                              tiles_sorted=tiles_sorted, count_dev=count_dev,
                              pair_live=pair_live)


def set_backward_chains(enabled: bool) -> bool:
    """Turn the backward's chained rows on or off for the rest of the process;
    returns the previous setting.  With them off the backward's results do not
    depend on which pairs share a 64-pair group (the cull flags, the capacity
    mode and the tile map then change no bit); with them on (the default,
    unless GSV_BWD_CHAIN=0 was set when the process first ran a backward) they
    agree to rounding.  Not in the reference."""
    prev = ctypes.c_int32(0)
    _call("set_backward_chains", 1 if enabled else 0, ctypes.byref(prev))
    return bool(prev.value)
