"""gsv_wave_timeline: the forward voxelize kernel records each workgroup's
start, end and tile while a buffer is registered, and nothing after it is
unregistered; the volume is unchanged by the recording."""
import ctypes

import numpy as np
import pytest
import torch

from gs_voxelizer import _lib, synthetic as S
from helpers import gpu_bin, gpu_project

pytestmark = pytest.mark.gpu


def test_forward_records_every_tile_once(device):
    import gs_voxelizer.cuda as _C
    L = _lib.load()
    work = S.make_gaussians(S.CONFIGS[1], seed=0)
    cfg = work.cfg
    pr, cn, tmin, tmax, nt = gpu_project(work, device)
    cum, I, ids, bins = gpu_bin(cfg.n, tmin, tmax, nt, cfg.vol)
    inten = work.intensities.to(device)
    ref = _C.voxelize_forward(cfg.vol, ids, bins, pr, cn, inten)
    T = int(np.prod(S.tile_grid(cfg.vol)))
    cap = (T + 63) // 64 * 64
    rec = torch.zeros((cap, 3), dtype=torch.int64, device=device)
    torch.cuda.synchronize()
    assert L.gsv_wave_timeline(0, ctypes.c_void_p(rec.data_ptr()), cap) == 0
    try:
        vol = _C.voxelize_forward(cfg.vol, ids, bins, pr, cn, inten)
        torch.cuda.synchronize()
    finally:
        assert L.gsv_wave_timeline(0, ctypes.c_void_p(0), 0) == 0
    assert torch.equal(vol, ref)
    r = rec.cpu().numpy()
    done = r[:, 0] > 0
    assert done.sum() == T
    assert (r[done, 1] >= r[done, 0]).all()
    np.testing.assert_array_equal(np.sort(r[done, 2]), np.arange(T))
    assert not r[~done].any()
    rec.zero_()
    _C.voxelize_forward(cfg.vol, ids, bins, pr, cn, inten)
    torch.cuda.synchronize()
    assert not rec.any()
