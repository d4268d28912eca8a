"""Caller workspaces need no alignment beyond 4 bytes: the kernels that read
them with 16-byte vector loads (the block-sum scan, the fused loss's final sum)
fall back to element loads when the pointer is not 16-byte aligned.  Checked by
calling the C-ABI with a workspace 4 bytes past an aligned allocation."""
import ctypes

import numpy as np
import pytest
import torch

from gs_voxelizer import synthetic as S
from helpers import np32, small_config

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("n", [5_000_011, 20_000_003])  # block sums: one tile, several
def test_cumsum_with_unaligned_workspace(device, n):
    import gs_voxelizer.cuda as _C
    g = np.random.default_rng(n)
    x = g.integers(0, 50, size=n).astype(np.int32)
    x[g.random(n) < 0.3] = 0
    src = torch.from_numpy(x).to(device)
    nb = ctypes.c_size_t(0)
    assert _C._L.gsv_scan_workspace_bytes(ctypes.c_int64(n), ctypes.byref(nb)) == 0
    ws = torch.empty((nb.value + 64,), device=device, dtype=torch.uint8)
    cum = torch.empty((n,), device=device, dtype=torch.int32)
    total = torch.empty((1,), device=device, dtype=torch.int64)
    ws_ptr = ctypes.c_void_p(ws.data_ptr() + 4)
    st = _C._L.gsv_cumsum_tiles_hit(ctypes.c_int32(n), _p(src), _p(cum), _p(total),
                                    ctypes.c_void_p(0), ws_ptr, ctypes.c_size_t(nb.value),
                                    _stream())
    assert st == 0
    torch.cuda.synchronize()
    ref = np.cumsum(x.astype(np.int64))
    np.testing.assert_array_equal(np32(cum), ref.astype(np.int32))
    assert int(total.item()) == int(ref[-1])


def test_fused_l1_loss_with_unaligned_workspace(device):
    import gs_voxelizer.cuda as _C
    work = S.make_gaussians(small_config(3, 3000, vol=(72, 64, 80)), seed=11)
    cfg = work.cfg
    w = work.to(device)
    target = S.phantom(work, device=device).contiguous()
    D, H, W = cfg.vol
    with torch.no_grad():
        pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(cfg.n, w.pos3d, w.scale3d, w.quat,
                                                            w.intensities, cfg.vol, cfg.world,
                                                            cfg.center)
        cum, total = _C.cumsum_tiles_hit(nt)
        I = int(total.item())
        ids, bins = _C.bin_and_sort_gaussians(cfg.n, I, tmin, tmax, cum, cfg.vol)
        vol_ref, loss_ref, sign_ref = _C.voxelize_forward_l1(cfg.vol, ids, bins, pr, cn,
                                                             w.intensities, target)
    nb = ctypes.c_size_t(0)
    assert _C._L.gsv_voxelize_fwd_l1_workspace_bytes(D, H, W, ctypes.byref(nb)) == 0
    ws = torch.empty((nb.value + 64,), device=device, dtype=torch.uint8)
    vol = torch.empty((D, H, W, 1), device=device)
    sign = torch.empty((D, H, W, 1), device=device, dtype=torch.int8)
    loss = torch.empty((), device=device)
    st = _C._L.gsv_voxelize_fwd_l1(D, H, W, 1, cfg.n, ctypes.c_int64(I), _p(ids), _p(bins),
                                   _p(pr), _p(cn), _p(w.intensities), _p(target), _p(vol),
                                   _p(sign), _p(loss), ctypes.c_void_p(0),
                                   ctypes.c_void_p(ws.data_ptr() + 4), ctypes.c_size_t(nb.value),
                                   _stream())
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(vol, vol_ref) and torch.equal(sign, sign_ref)
    # the same partials summed in another order (element loads, one running sum)
    assert abs(loss.item() - loss_ref.item()) <= 1e-6 * abs(loss_ref.item())
    expect = (vol_ref[..., 0].double() - target.double()).abs().mean().item()
    assert abs(loss.item() - expect) <= 1e-5 * expect
