"""Differentiable voxelization of projected Gaussians into a (D, H, W, C) grid.

Drop-in for gs_voxelizer/voxelize.py of the reference (lines 14-173): same
function, arguments, empty-input behaviour and autograd outputs.  The prefix sum
of tile counts, binning, forward and backward run in libgsvox.so.

The reference reads the intersection count back to the host before binning
(voxelize.py:87-88), which idles the GPU for a round trip every forward.  Here
the first forward on a device does the same and records a capacity; later
forwards launch binning and the forward kernel at that capacity with the count
left on the device (the prefix-sum kernel also writes it into pinned host
memory, so no copy is enqueued), and check it after the launches.  A count
above the capacity (the scene grew) reruns binning and the forward with the
exact count and raises the capacity; results are identical either way.  GSV_SYNC_COUNT=1 restores the reference's host read.
"""
import os
import threading
from typing import Tuple

import torch
from torch import Tensor
from torch.autograd import Function

import gs_voxelizer.cuda as _C

_INT32_MAX = 2**31 - 1
_capacity = {}  # device index -> intersection capacity of the speculative path
_SLOTS = 64  # pinned count slots per device, taken in turn by the forwards
_slot_pool = {}  # device index -> [pinned int64 (_SLOTS,), next slot]
_slot_lock = threading.Lock()
_capture = threading.local()  # .counts: [(pinned count, capacity)] of the capture under way


def _grow(count: int) -> int:
    return min(_INT32_MAX, count + count // 4 + 4096)


def _speculate() -> bool:
    return os.environ.get("GSV_SYNC_COUNT", "0") != "1"


_SPIN_READS = 1 << 21  # reads of the pinned count before falling back to a device sync


def _count_slot(dev: torch.device) -> Tensor:
    """A pinned (1,) int64 for one eager forward's pair count.  Slots are taken
    in turn from a per-device pool, so forwards running at the same time on
    other streams or threads write their own (a forward reads its slot before it
    returns, long before the pool comes round to it again)."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    with _slot_lock:
        pool = _slot_pool.get(key)
        if pool is None:
            pool = [torch.empty((_SLOTS,), dtype=torch.int64, pin_memory=True), 0]
            _slot_pool[key] = pool
        i = pool[1]
        pool[1] = (i + 1) % _SLOTS
    return pool[0][i:i + 1]


def begin_capture(max_forwards: int = 16) -> None:
    """Prepare the graph capture that follows on this thread: pinned counts
    (allocated here, outside the capture) for up to `max_forwards` captured
    forwards, each written by its prefix-sum kernel at every replay."""
    _capture.free = [torch.empty((1,), dtype=torch.int64, pin_memory=True)
                     for _ in range(max(int(max_forwards), 1))]
    _capture.counts = []


def end_capture():
    """[(pinned (1,) int64 count, capacity the arrays were captured with)], one
    per forward captured since begin_capture()."""
    counts = getattr(_capture, "counts", None) or []
    _capture.counts = _capture.free = None
    return counts


def capacity(device=None):
    """The intersection capacity recorded for `device` (None before the first
    forward on it)."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    return _capacity.get(dev.index if dev.index is not None else torch.cuda.current_device())


def _await_count(host: Tensor, dev: torch.device) -> int:
    """The pair count the prefix-sum kernel writes into pinned memory (-1 until
    then).  Polling it, rather than recording an event behind the kernel, keeps
    an extra completion packet out of the queue; the kernels queued after the
    scan keep the GPU busy meanwhile."""
    for _ in range(_SPIN_READS):
        v = int(host[0])
        if v >= 0:
            return v
    torch.cuda.synchronize(dev)
    v = int(host[0])
    if v < 0:
        raise RuntimeError("gs_voxelizer: the intersection count was not written")
    return v


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


def _bin_and_forward(num_gaussians, vol_size_voxel, tile_min, tile_max, num_tiles_hit, fwd):
    """Prefix sum, binning and `fwd(gaussian_ids_sorted, tile_bins)` for a
    non-empty Gaussian set.  Returns (num_intersects, ids, tile_bins, tiles, cum,
    fwd's result, count_dev), tiles being the tile id of each sorted pair (for
    the backward); ids and tiles are None when there are no intersections.

    Under graph capture nothing is read back: the arrays keep the recorded
    capacity, num_intersects is that capacity and count_dev (the live count on
    the device) bounds the backward; each replay's count lands in a pinned
    buffer of this forward's own, listed by end_capture() with the capacity for
    the caller to check (gs_voxelizer.graph does)."""
    dev = num_tiles_hit.device
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    cap = _capacity.get(key) if _speculate() else None
    if torch.cuda.is_current_stream_capturing():
        if cap is None:
            raise RuntimeError(
                "gs_voxelizer: run the step once outside graph capture first (it records the "
                "intersection capacity the captured arrays are sized for), and leave "
                "GSV_SYNC_COUNT unset")
        free = getattr(_capture, "free", None)
        if not free:
            raise RuntimeError(
                "gs_voxelizer: capture voxelization through gs_voxelizer.graph.CapturedStep "
                "(it checks every replay's intersection count), at most 16 forwards a step")
        host = free.pop()
        _capture.counts.append((host, cap))
        cum_tiles_hit, total, ids_cap, tile_bins, tiles_cap = _C.cumsum_bin_and_sort_device_count(
            num_gaussians, cap, num_tiles_hit.contiguous(), tile_min, tile_max, vol_size_voxel,
            total_host=host, return_tiles=True)
        return (cap, ids_cap, tile_bins, tiles_cap, cum_tiles_hit, fwd(ids_cap, tile_bins),
                total)
    if cap is not None:
        # launch at the recorded capacity; the scan writes the count into pinned
        # memory meanwhile
        host = _count_slot(dev)
        host.fill_(-1)
        # the prefix sum and the binning in one native call (four launches on
        # the bucket path); the scan writes the count into pinned memory
        cum_tiles_hit, total, ids_cap, tile_bins, tiles_cap = _C.cumsum_bin_and_sort_device_count(
            num_gaussians, cap, num_tiles_hit.contiguous(), tile_min, tile_max, vol_size_voxel,
            total_host=host, return_tiles=True)
        result = fwd(ids_cap, tile_bins)
        num_intersects = _await_count(host, dev)
        if num_intersects <= cap:
            if num_intersects < cap // 4:
                _capacity[key] = _grow(num_intersects)
            if num_intersects < 1:
                return 0, None, tile_bins, None, cum_tiles_hit, result, None
            return (num_intersects, ids_cap[:num_intersects], tile_bins,
                    tiles_cap[:num_intersects], cum_tiles_hit, result, None)
    else:
        cum_tiles_hit, total = _C.cumsum_tiles_hit(num_tiles_hit.contiguous())
        num_intersects = int(total.item())
    if num_intersects > _INT32_MAX:
        raise RuntimeError(
            f"gs_voxelizer: {num_intersects} tile intersections overflow the int32 layout")
    if _speculate():
        _capacity[key] = _grow(num_intersects)
    if num_intersects < 1:
        return 0, None, None, None, cum_tiles_hit, None, None
    # first call on the device, host read requested, or the capacity overflowed
    ids, tile_bins, tiles = _C.bin_and_sort_gaussians(
        num_gaussians, num_intersects, tile_min.contiguous(), tile_max.contiguous(),
        cum_tiles_hit, vol_size_voxel, return_tiles=True)
    return num_intersects, ids, tile_bins, tiles, cum_tiles_hit, fwd(ids, tile_bins), None


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
        C = intensities.shape[-1]
        boxes = ()
        gaussian_ids_sorted = tile_bins = None
        ctx.num_intersects = 0
        if num_gaussians > 0:
            def fwd(ids, bins):
                live = torch.empty(ids.numel(), device=dev, dtype=torch.uint8)
                return _C.voxelize_forward(vol_size_voxel, ids, bins, pos3d_radii, conics,
                                           intensities, pair_live=live), live
            I, gaussian_ids_sorted, tile_bins, tiles, cum_tiles_hit, res, count = _bin_and_forward(
                num_gaussians, vol_size_voxel, tile_min, tile_max, num_tiles_hit, fwd)
            ctx.num_intersects = I
            if I >= 1:
                out, live = res
                # the backward reduces per-pair partials in duplication order (no
                # atomics), takes each sorted pair's tile from the binning and
                # skips the pairs the forward culled
                boxes = (tile_min.contiguous(), tile_max.contiguous(), cum_tiles_hit, tiles, live)
                if count is not None:  # captured: capacity-sized arrays, live count on device
                    boxes += (count,)
        if ctx.num_intersects < 1:
            out = torch.zeros(D, H, W, C, device=dev, dtype=pos3d_radii.dtype)
            gaussian_ids_sorted = torch.zeros(0, 1, device=dev, dtype=torch.int32)
            tile_bins = torch.zeros(0, 3, device=dev, dtype=torch.int32)
            boxes = ()
        ctx.set_materialize_grads(False)  # an unused volume needs no zero-filled gradient
        ctx.save_for_backward(pos3d_radii, conics, intensities, gaussian_ids_sorted, tile_bins,
                              *boxes)
        return out

    @staticmethod
    def backward(ctx, vol_grad):
        vol_size_voxel = ctx.vol_size_voxel
        saved = ctx.saved_tensors
        pos3d_radii, conics, intensities, gaussian_ids_sorted, tile_bins = saved[:5]
        boxes, tiles = saved[5:8], (saved[8] if len(saved) > 8 else None)
        live = saved[9] if len(saved) > 9 else None
        count = saved[10] if len(saved) > 10 else None
        if ctx.num_intersects < 1 or vol_grad is None:
            pos3d_grad = torch.zeros_like(pos3d_radii)
            conics_grad = torch.zeros_like(conics)
            intensities_grad = torch.zeros_like(intensities)
        else:
            fn = (_C.voxelize_backward_per_gaussian if ctx.use_per_gaussian_backward
                  else _C.voxelize_backward)
            pos3d_grad, conics_grad, intensities_grad = fn(
                vol_size_voxel, gaussian_ids_sorted, tile_bins, pos3d_radii, conics, intensities,
                vol_grad.contiguous(), *boxes, tiles_sorted=tiles, count_dev=count, pair_live=live)
        return pos3d_grad, conics_grad, intensities_grad, None, None, None, None, None


def voxelize_gaussians_l1_loss(
    pos3d_radii: Tensor,
    conics: Tensor,
    intensities: Tensor,
    vol_size_voxel: Tuple[int, int, int],
    tile_min: Tensor,
    tile_max: Tensor,
    num_tiles_hit: Tensor,
    target: Tensor,
    use_per_gaussian_backward: bool = True,
) -> Tuple[Tensor, Tensor]:
    """voxelize_gaussians fused with the L1 loss of the reference's training loop.

    Returns (loss, volume) with loss = torch.nn.functional.l1_loss(volume, target)
    (mean over all elements).  The backward forms dL/dvolume = sgn(volume -
    target) * grad / numel inside the voxelization backward instead of
    materialising it (and the loss inside the forward kernel), which is the same
    gradient, bit for bit, as the unfused sequence.  `target` has the volume's
    (D, H, W, C) shape, or (D, H, W) for one channel.  The returned volume is
    differentiable too; a gradient reaching it from other uses is added.
    The loss equals torch's up to float summation order.
    """
    return _VoxelizeL1.apply(
        pos3d_radii.contiguous(),
        conics.contiguous(),
        intensities.contiguous(),
        vol_size_voxel,
        tile_min,
        tile_max,
        num_tiles_hit,
        target.contiguous(),
        use_per_gaussian_backward,
    )


class _VoxelizeL1(Function):
    @staticmethod
    def forward(ctx, pos3d_radii, conics, intensities, vol_size_voxel, tile_min, tile_max,
                num_tiles_hit, target, use_per_gaussian_backward=True):
        if intensities.dim() == 1:
            intensities = intensities.unsqueeze(-1)
        num_gaussians = pos3d_radii.size(-2)
        ctx.vol_size_voxel = vol_size_voxel
        ctx.use_per_gaussian_backward = use_per_gaussian_backward
        dev = pos3d_radii.device
        D, H, W = (int(v) for v in vol_size_voxel)
        C = intensities.shape[-1]
        def fwd(ids, bins):
            live = torch.empty(ids.numel(), device=dev, dtype=torch.uint8)
            return _C.voxelize_forward_l1(vol_size_voxel, ids, bins, pos3d_radii, conics,
                                          intensities, target, pair_live=live) + (live,)
        boxes = ()
        ctx.num_intersects = 0
        if num_gaussians > 0:
            I, ids, tile_bins, tiles, cum_tiles_hit, res, count = _bin_and_forward(
                num_gaussians, vol_size_voxel, tile_min, tile_max, num_tiles_hit, fwd)
            ctx.num_intersects = I
            if I >= 1:
                boxes = (tile_min.contiguous(), tile_max.contiguous(), cum_tiles_hit, tiles,
                         res[3])
                if count is not None:  # captured: capacity-sized arrays, live count on device
                    boxes += (count,)
        if ctx.num_intersects < 1:
            # no Gaussian touches the volume: it is zero, the loss mean(|target|)
            empty_ids = torch.zeros(0, device=dev, dtype=torch.int32)
            Tx, Ty, Tz = ((int(v) + 7) // 8 for v in (W, H, D))
            bins = torch.zeros(Tx * Ty * Tz, 2, device=dev, dtype=torch.int32)
            res = fwd(empty_ids, bins)
            ids, tile_bins, boxes = empty_ids, bins, ()
        volume, loss, sign = res[:3]
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(pos3d_radii, conics, intensities, ids, tile_bins, sign, *boxes)
        return loss, volume

    @staticmethod
    def backward(ctx, grad_loss, grad_volume):
        saved = ctx.saved_tensors
        pos3d_radii, conics, intensities, ids, tile_bins, sign = saved[:6]
        boxes, tiles = saved[6:9], (saved[9] if len(saved) > 9 else None)
        live = saved[10] if len(saved) > 10 else None
        count = saved[11] if len(saved) > 11 else None
        if ctx.num_intersects < 1 or (grad_loss is None and grad_volume is None):
            z = (torch.zeros_like(pos3d_radii), torch.zeros_like(conics),
                 torch.zeros_like(intensities))
        else:
            if grad_loss is None:
                grad_loss = torch.zeros((), device=sign.device, dtype=torch.float32)
            z = _C.voxelize_backward_l1(
                ctx.vol_size_voxel, ids, tile_bins, pos3d_radii, conics, intensities, sign,
                grad_loss.contiguous(),
                grad_volume.contiguous() if grad_volume is not None else None, *boxes,
                per_gaussian=ctx.use_per_gaussian_backward, tiles_sorted=tiles, count_dev=count,
                pair_live=live)
        return z[0], z[1], z[2], None, None, None, None, None, None
