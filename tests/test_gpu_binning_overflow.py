"""Binning with a pair count past 2^31 and a small capacity stays inside its arrays.

70,000 Gaussians whose boxes each cover the whole 32^3-tile grid of a 256^3
volume sum to 2,293,760,000 (tile, Gaussian) pairs, past int32.  The pair
counts per bucket are int32 sums; their prefix over buckets passes 2^31 from
the ~240th of the 256 buckets on, so a binning that used it as an int32 offset
would read and write before its arrays.  Called with a capacity of 2^20 (the
speculative path of a caller whose scene grew), the combined prefix sum and
binning, and the plain device-count binning fed the wrapped int32 prefix sum,
must return, report the full count, and leave guard words around every output
and the workspace untouched.  The outputs past the capacity are unspecified
(the caller bins again with the count), so only the count is compared.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

GUARD_I32 = 0x5A5A5A5A
GUARD_U8 = 0x5A
PAD = 1024  # guard words on each side (16-byte alignment kept)


def _guarded(n, dtype, device, fill):
    buf = torch.full((n + 2 * PAD,), fill, dtype=dtype, device=device)
    return buf, buf[PAD:PAD + n]


def _intact(buf, n, fill):
    return bool((buf[:PAD] == fill).all()) and bool((buf[PAD + n:] == fill).all())


def test_pair_count_past_int32_with_small_capacity(device):
    import gs_voxelizer.cuda as _C
    D = H = W = 256
    T = 32 ** 3
    n = 70_000
    cap = 1 << 20
    print(f"binning overflow: n={n}, pairs={n * T}, capacity={cap}", flush=True)
    i32 = dict(device=device, dtype=torch.int32)
    tmin = torch.zeros((n, 3), **i32)
    tmax = torch.full((n, 3), 32, **i32)
    nth = torch.full((n,), T, **i32)
    cum = torch.empty((n,), **i32)
    total = torch.full((1,), -1, device=device, dtype=torch.int64)
    ids_buf, ids = _guarded(cap, torch.int32, device, GUARD_I32)
    tiles_buf, tiles = _guarded(cap, torch.int32, device, GUARD_I32)
    bins_buf, bins = _guarded(2 * T, torch.int32, device, GUARD_I32)
    nbytes = ctypes.c_size_t(0)
    _C._call("cumsum_bin_workspace_bytes", n, cap, D, H, W, ctypes.byref(nbytes))
    ws_buf, ws = _guarded(nbytes.value, torch.uint8, device, GUARD_U8)
    null = ctypes.c_void_p(0)
    with torch.cuda.device(device):
        _C._call("cumsum_bin_and_sort_device_count", n, cap, _C._ptr(nth), _C._ptr(tmin),
                 _C._ptr(tmax), D, H, W, _C._ptr(cum), _C._ptr(total), null, _C._ptr(ws),
                 nbytes.value, _C._ptr(ids), _C._ptr(bins), _C._ptr(tiles), _C._stream(device))
    torch.cuda.synchronize()
    assert int(total.item()) == n * T
    for name, buf, size, fill in (("ids", ids_buf, cap, GUARD_I32),
                                  ("tiles", tiles_buf, cap, GUARD_I32),
                                  ("tile_bins", bins_buf, 2 * T, GUARD_I32),
                                  ("workspace", ws_buf, nbytes.value, GUARD_U8)):
        assert _intact(buf, size, fill), f"combined call wrote outside {name}"

    # the plain device-count binning, fed the int32 prefix sum that wrapped
    # past 2^31 and the int64 count
    _C._call("bin_workspace_bytes", n, cap, D, H, W, ctypes.byref(nbytes))
    ws_buf, ws = _guarded(nbytes.value, torch.uint8, device, GUARD_U8)
    for buf, fill in ((ids_buf, GUARD_I32), (tiles_buf, GUARD_I32), (bins_buf, GUARD_I32)):
        buf.fill_(fill)
    with torch.cuda.device(device):
        _C._call("bin_and_sort_device_count", n, cap, _C._ptr(total), _C._ptr(tmin),
                 _C._ptr(tmax), _C._ptr(cum), D, H, W, _C._ptr(ws), nbytes.value,
                 _C._ptr(ids), _C._ptr(bins), _C._ptr(tiles), _C._stream(device))
    torch.cuda.synchronize()
    for name, buf, size, fill in (("ids", ids_buf, cap, GUARD_I32),
                                  ("tiles", tiles_buf, cap, GUARD_I32),
                                  ("tile_bins", bins_buf, 2 * T, GUARD_I32),
                                  ("workspace", ws_buf, nbytes.value, GUARD_U8)):
        assert _intact(buf, size, fill), f"device-count call wrote outside {name}"
