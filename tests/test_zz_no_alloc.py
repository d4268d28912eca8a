"""gsv_bin_and_sort_noalloc (binning with the library's fixed per-GPU scratch,
no allocation) against gsv_bin_and_sort (caller workspace), through the C ABI:
bit-exact outputs on two calls in a row, the second with a smaller problem
(the scratch keeps the first call's contents), then the oracle on the smaller
one, and the size limit refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gs_voxelizer import _lib, synthetic as S
from helpers import gpu_project, small_config

pytestmark = pytest.mark.gpu

MAX_PAIRS = 4194304  # GSV_NOALLOC_MAX_INTERSECTIONS


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _inputs(work, device):
    import gs_voxelizer.cuda as _C
    pr, cn, tmin, tmax, nt = gpu_project(work, device)
    cum, total = _C.cumsum_tiles_hit(nt)
    return tmin, tmax, cum, int(total.item())


def _bin_both(work, device):
    L = _lib.load()
    cfg = work.cfg
    n = work.pos3d.shape[0]
    D, H, W = cfg.vol
    T = int(np.prod(S.tile_grid(cfg.vol)))
    tmin, tmax, cum, I = _inputs(work, device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws_bytes = ctypes.c_size_t(0)
    assert L.gsv_bin_workspace_bytes(n, I, D, H, W, ctypes.byref(ws_bytes)) == 0
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=device)
    out = []
    for noalloc in (False, True):
        # poisoned outputs: every entry must be written
        ids = torch.full((max(I, 1),), -7, dtype=torch.int32, device=device)
        tiles = torch.full((max(I, 1),), -7, dtype=torch.int32, device=device)
        bins = torch.full((T, 2), -7, dtype=torch.int32, device=device)
        if noalloc:
            st = L.gsv_bin_and_sort_noalloc(n, I, _ptr(tmin), _ptr(tmax), _ptr(cum), D, H, W,
                                            _ptr(ids), _ptr(bins), _ptr(tiles), stream)
        else:
            st = L.gsv_bin_and_sort(n, I, _ptr(tmin), _ptr(tmax), _ptr(cum), D, H, W, _ptr(ws),
                                    ws_bytes, _ptr(ids), _ptr(bins), _ptr(tiles), stream)
        assert st == 0, L.gsv_status_string(st)
        torch.cuda.synchronize()
        out.append((ids[:I].cpu().numpy(), bins.cpu().numpy(), tiles[:I].cpu().numpy()))
    return I, out, (tmin, tmax, cum)


def test_noalloc_binning_matches_workspace_binning_twice(device, binning_path):
    """Through each sort path (GSV_BINNING) and the library's own choice."""
    works = [("cfg3_full", S.make_gaussians(S.CONFIGS[3], seed=0)),
             ("cfg1_smaller", S.make_gaussians(S.CONFIGS[1], seed=1))]
    sizes = []
    for name, work in works:
        print(f"noalloc binning: {name}, path {binning_path}", flush=True)
        I, ((ids_a, bins_a, tiles_a), (ids_b, bins_b, tiles_b)), (tmin, tmax, cum) = \
            _bin_both(work, device)
        assert 0 < I <= MAX_PAIRS
        sizes.append(I)
        np.testing.assert_array_equal(ids_b, ids_a, err_msg=f"{name}: gaussian_ids_sorted")
        np.testing.assert_array_equal(bins_b, bins_a, err_msg=f"{name}: tile_bins")
        np.testing.assert_array_equal(tiles_b, tiles_a, err_msg=f"{name}: tiles_sorted")
    assert sizes[1] < sizes[0]
    # the smaller problem against the oracle as well
    cfg = works[1][1].cfg
    n = works[1][1].pos3d.shape[0]
    ref_ids, ref_bins = O.bin_and_sort(n, sizes[1], tmin.cpu().numpy(), tmax.cpu().numpy(),
                                       cum.cpu().numpy(), cfg.vol)
    np.testing.assert_array_equal(ids_b, ref_ids)
    np.testing.assert_array_equal(bins_b, ref_bins)


def test_noalloc_binning_empty_and_limit(device):
    """No pairs: tile_bins zero-filled, nothing else touched.  One pair beyond
    the limit: refused with GSV_ERR_SCRATCH_TOO_SMALL."""
    L = _lib.load()
    work = S.make_gaussians(small_config(1, 64, vol=(16, 24, 32)), seed=2)
    tmin, tmax, cum, I = _inputs(work, device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    bins = torch.full((2 * 3 * 4, 2), -7, dtype=torch.int32, device=device)
    st = L.gsv_bin_and_sort_noalloc(64, 0, _ptr(tmin), _ptr(tmax), _ptr(cum), 16, 24, 32,
                                    ctypes.c_void_p(0), _ptr(bins), ctypes.c_void_p(0), stream)
    assert st == 0
    torch.cuda.synchronize()
    assert int(bins.abs().sum()) == 0
    st = L.gsv_bin_and_sort_noalloc(64, MAX_PAIRS + 1, _ptr(tmin), _ptr(tmax), _ptr(cum),
                                    16, 24, 32, _ptr(bins), _ptr(bins), ctypes.c_void_p(0),
                                    stream)
    assert st == 6


def test_noalloc_falls_back_to_lsd_when_bucket_counts_do_not_fit(device):
    """3.5M one-tile Gaussians on a 512^3 grid (18-bit keys, 1024 buckets): the
    bucket path's counts, 1024 per 256 Gaussians (56 MB), exceed the scratch
    array, so the allocation-free entry takes the LSD passes while the
    workspace entry takes the bucket path; both give the oracle's bits."""
    L = _lib.load()
    D = H = W = 512
    n = 3_500_000
    g = torch.Generator().manual_seed(5)
    tmin = torch.randint(0, 64, (n, 3), generator=g, dtype=torch.int32)
    tmax = tmin + 1
    cum = torch.arange(1, n + 1, dtype=torch.int32)
    I = n
    assert I <= MAX_PAIRS
    T = 64 ** 3
    dev = [t.to(device) for t in (tmin, tmax, cum)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws_bytes = ctypes.c_size_t(0)
    assert L.gsv_bin_workspace_bytes(n, I, D, H, W, ctypes.byref(ws_bytes)) == 0
    assert ws_bytes.value > 52431104  # the bucket layout alone outgrows the scratch
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=device)
    out = []
    for noalloc in (False, True):
        print(f"noalloc LSD fallback: noalloc={noalloc}", flush=True)
        ids = torch.full((I,), -7, dtype=torch.int32, device=device)
        tiles = torch.full((I,), -7, dtype=torch.int32, device=device)
        bins = torch.full((T, 2), -7, dtype=torch.int32, device=device)
        if noalloc:
            st = L.gsv_bin_and_sort_noalloc(n, I, _ptr(dev[0]), _ptr(dev[1]), _ptr(dev[2]), D, H,
                                            W, _ptr(ids), _ptr(bins), _ptr(tiles), stream)
        else:
            st = L.gsv_bin_and_sort(n, I, _ptr(dev[0]), _ptr(dev[1]), _ptr(dev[2]), D, H, W,
                                    _ptr(ws), ws_bytes, _ptr(ids), _ptr(bins), _ptr(tiles),
                                    stream)
        assert st == 0, L.gsv_status_string(st)
        torch.cuda.synchronize()
        out.append((ids.cpu().numpy(), bins.cpu().numpy(), tiles.cpu().numpy()))
    for a, b, what in zip(out[0], out[1], ("gaussian_ids_sorted", "tile_bins", "tiles_sorted")):
        np.testing.assert_array_equal(b, a, err_msg=what)
    ref_ids, ref_bins = O.bin_and_sort(n, I, tmin.numpy(), tmax.numpy(), cum.numpy(), (D, H, W))
    np.testing.assert_array_equal(out[1][0], ref_ids)
    np.testing.assert_array_equal(out[1][1], ref_bins)
