"""numpy front-end of the C oracle (``liboracle.so``). Test infrastructure only.

Every function takes and returns contiguous numpy arrays with the layouts of the
reference API: pos3d/scale3d (N,3) f32, quat (N,4) f32 [w,x,y,z], intensities
(N,C) f32, volume tuples (z, y, x), pos3d_radii (N,4), conics (N,6),
tile_min/tile_max (N,3) i32, num_tiles_hit (N,) i32, gaussian_ids_sorted (I,)
i32, tile_bins (T,2) i32, volume (D,H,W,C) f32.
"""
import ctypes
import os
import subprocess

import numpy as np

__all__ = [
    "lib", "build", "num_threads", "logf", "f2i_sat", "project_fwd", "project_bwd",
    "cumsum", "bin_and_sort", "voxelize_fwd", "voxelize_bwd", "tile_grid", "pipeline",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_c_int, _c_float, _c_i64 = ctypes.c_int, ctypes.c_float, ctypes.c_int64


def build():
    """Compile gsv_oracle.c into liboracle.so (gcc, no GPU needed)."""
    subprocess.check_call(["sh", os.path.join(_HERE, "build_oracle.sh")])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        L.orc_project_fwd.argtypes = [_c_int, _c_int, _f32p, _f32p, _f32p, _f32p,
                                      _c_int, _c_int, _c_int, _c_float, _c_float, _c_float,
                                      _c_float, _c_float, _c_float,
                                      _f32p, _f32p, _i32p, _i32p, _i32p]
        L.orc_project_bwd.argtypes = [_c_int, _f32p, _f32p, _f32p, _c_int, _c_int, _c_int,
                                      _c_float, _c_float, _c_float, _c_float, _c_float, _c_float,
                                      _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_cumsum_i32.argtypes = [_c_int, _i32p, _i32p]
        L.orc_cumsum_i32.restype = None
        L.orc_bin_and_sort.argtypes = [_c_int, _c_i64, _i32p, _i32p, _i32p, _c_int, _c_int, _c_int,
                                       _i32p, _i32p, ctypes.c_void_p]
        L.orc_voxelize_fwd.argtypes = [_c_int, _c_int, _c_int, _c_int, _i32p, _i32p, _f32p, _f32p,
                                       _f32p, _f32p, ctypes.c_void_p, _c_i64, _c_i64]
        L.orc_voxelize_bwd.argtypes = [_c_int, _c_int, _c_int, _c_int, _c_int, _i32p, _i32p, _f32p,
                                       _f32p, _f32p, _f32p, _f32p, _f32p, _f32p] + \
            [ctypes.c_void_p] * 6 + [_c_i64, _c_i64]
        L.orc_logf.argtypes = [_c_float]
        L.orc_logf.restype = _c_float
        L.orc_f2i_sat.argtypes = [_c_float]
        L.orc_f2i_sat.restype = _c_int
        L.orc_num_threads.restype = _c_int
        _lib = L
    return _lib


def num_threads():
    return lib().orc_num_threads()


def logf(x):
    return lib().orc_logf(float(x))


def f2i_sat(x):
    return lib().orc_f2i_sat(float(x))


def _f32(a, cols=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    if cols is not None:
        a = a.reshape(-1, cols)
    return a


def _i32(a, cols=None):
    a = np.ascontiguousarray(a, dtype=np.int32)
    if cols is not None:
        a = a.reshape(-1, cols)
    return a


def tile_grid(vol_size_voxel):
    """(Tx, Ty, Tz) for a (D, H, W) volume, bindings.cu:70-74."""
    D, H, W = (int(v) for v in vol_size_voxel)
    return (W + 7) // 8, (H + 7) // 8, (D + 7) // 8


def _check(rc, name):
    if rc != 0:
        raise RuntimeError(f"oracle {name} failed with status {rc}")


def project_fwd(pos3d, scale3d, quat, intensities, vol_size_voxel, vol_size_world, vol_center_pos):
    pos3d, scale3d, quat = _f32(pos3d, 3), _f32(scale3d, 3), _f32(quat, 4)
    n = pos3d.shape[0]
    intensities = _f32(intensities).reshape(n, -1)
    C = intensities.shape[1]
    D, H, W = (int(v) for v in vol_size_voxel)
    wz, wy, wx = (float(v) for v in vol_size_world)
    cz, cy, cx = (float(v) for v in vol_center_pos)
    pr = np.empty((n, 4), np.float32)
    cn = np.empty((n, 6), np.float32)
    tmin = np.empty((n, 3), np.int32)
    tmax = np.empty((n, 3), np.int32)
    nt = np.empty((n,), np.int32)
    _check(lib().orc_project_fwd(n, C, pos3d, scale3d, quat, intensities, D, H, W, wz, wy, wx,
                                 cz, cy, cx, pr, cn, tmin, tmax, nt), "project_fwd")
    return pr, cn, tmin, tmax, nt


def project_bwd(pos3d, scale3d, quat, vol_size_voxel, vol_size_world, vol_center_pos,
                dpos_radii, dconics, pos_radii):
    pos3d, scale3d, quat = _f32(pos3d, 3), _f32(scale3d, 3), _f32(quat, 4)
    n = pos3d.shape[0]
    D, H, W = (int(v) for v in vol_size_voxel)
    wz, wy, wx = (float(v) for v in vol_size_world)
    cz, cy, cx = (float(v) for v in vol_center_pos)
    dp = np.empty((n, 3), np.float32)
    ds = np.empty((n, 3), np.float32)
    dq = np.empty((n, 4), np.float32)
    _check(lib().orc_project_bwd(n, pos3d, scale3d, quat, D, H, W, wz, wy, wx, cz, cy, cx,
                                 _f32(dpos_radii, 4), _f32(dconics, 6), _f32(pos_radii, 4),
                                 dp, ds, dq), "project_bwd")
    return dp, ds, dq


def cumsum(num_tiles_hit):
    x = _i32(num_tiles_hit).reshape(-1)
    out = np.empty_like(x)
    lib().orc_cumsum_i32(x.shape[0], x, out)
    return out


def bin_and_sort(num_gaussians, num_intersects, tile_min, tile_max, cum_tiles_hit, vol_size,
                 return_keys=False):
    tmin, tmax = _i32(tile_min, 3), _i32(tile_max, 3)
    cum = _i32(cum_tiles_hit).reshape(-1)
    D, H, W = (int(v) for v in vol_size)
    Tx, Ty, Tz = tile_grid(vol_size)
    T = Tx * Ty * Tz
    I = max(int(num_intersects), 0)
    ids = np.empty((I,), np.int32)
    bins = np.empty((T, 2), np.int32)
    keys = np.empty((I,), np.int32) if return_keys else None
    _check(lib().orc_bin_and_sort(int(num_gaussians), int(num_intersects), tmin, tmax, cum,
                                  D, H, W, ids, bins,
                                  keys.ctypes.data_as(ctypes.c_void_p) if return_keys else None),
           "bin_and_sort")
    return (ids, bins, keys) if return_keys else (ids, bins)


def voxelize_fwd(vol_size, ids_sorted, tile_bins, pos_radii, conics, intensities,
                 tile_range=None, with_amb=False):
    """(D,H,W,C) volume; with ``with_amb`` also the per-voxel sum of |I*alpha|
    over gate-ambiguous evaluations (see gate_ambiguous in gsv_oracle.c)."""
    D, H, W = (int(v) for v in vol_size)
    pr = _f32(pos_radii, 4)
    n = pr.shape[0]
    I = _f32(intensities).reshape(n, -1)
    C = I.shape[1]
    out = np.zeros((D, H, W, C), np.float32)
    amb = np.zeros((D, H, W, C), np.float32) if with_amb else None
    bins = _i32(tile_bins, 2)
    t0, t1 = tile_range if tile_range is not None else (0, bins.shape[0])
    _check(lib().orc_voxelize_fwd(D, H, W, C, _i32(ids_sorted).reshape(-1), bins, pr,
                                  _f32(conics, 6), I, out,
                                  amb.ctypes.data_as(ctypes.c_void_p) if with_amb else None,
                                  int(t0), int(t1)), "voxelize_fwd")
    return (out, amb) if with_amb else out


def voxelize_bwd(vol_size, ids_sorted, tile_bins, pos_radii, conics, intensities, vol_grad,
                 tile_range=None, diagnostics=False):
    """Returns (dpos_radii (N,4), dconics (N,6), dintens (N,C)).  With
    ``diagnostics`` returns (grads, abs_sums, ambiguous_sums), each a triple in
    the same layout: per element the sum of |term| over contributing voxels
    (conditioning) and over gate-ambiguous evaluations."""
    D, H, W = (int(v) for v in vol_size)
    pr = _f32(pos_radii, 4)
    n = pr.shape[0]
    I = _f32(intensities).reshape(n, -1)
    C = I.shape[1]
    g = _f32(vol_grad).reshape(D, H, W, C)
    bins = _i32(tile_bins, 2)
    t0, t1 = tile_range if tile_range is not None else (0, bins.shape[0])
    trip = lambda: (np.empty((n, 4), np.float32), np.empty((n, 6), np.float32),
                    np.empty((n, C), np.float32))
    grads, absum, amb = trip(), (trip() if diagnostics else None), (trip() if diagnostics else None)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    extra = [ptr(absum[0]), ptr(absum[1]), ptr(absum[2]), ptr(amb[0]), ptr(amb[1]),
             ptr(amb[2])] if diagnostics else [None] * 6
    _check(lib().orc_voxelize_bwd(D, H, W, C, n, _i32(ids_sorted).reshape(-1), bins, pr,
                                  _f32(conics, 6), I, g, grads[0], grads[1], grads[2], *extra,
                                  int(t0), int(t1)), "voxelize_bwd")
    return (grads, absum, amb) if diagnostics else grads


def pipeline(pos3d, scale3d, quat, intensities, vol_size_voxel, vol_size_world, vol_center_pos,
             vol_grad=None):
    """Whole forward (and, given vol_grad, backward) on the CPU, as the
    reference's Python layer sequences it (optim_to_render.py:56-149,
    voxelize.py:55-173). Returns a dict of every intermediate."""
    pr, cn, tmin, tmax, nt = project_fwd(pos3d, scale3d, quat, intensities, vol_size_voxel,
                                         vol_size_world, vol_center_pos)
    n = pr.shape[0]
    I = _f32(intensities).reshape(n, -1)
    cum = cumsum(nt)
    n_isect = int(cum[-1]) if n > 0 else 0
    ids, bins = bin_and_sort(n, n_isect, tmin, tmax, cum, vol_size_voxel)
    vol = voxelize_fwd(vol_size_voxel, ids, bins, pr, cn, I)
    out = dict(pos3d_radii=pr, conics=cn, tile_min=tmin, tile_max=tmax, num_tiles_hit=nt,
               cum_tiles_hit=cum, num_intersects=n_isect, gaussian_ids_sorted=ids, tile_bins=bins,
               volume=vol)
    if vol_grad is not None:
        dpr, dcn, dI = voxelize_bwd(vol_size_voxel, ids, bins, pr, cn, I, vol_grad)
        dpos, dscale, dquat = project_bwd(pos3d, scale3d, quat, vol_size_voxel, vol_size_world,
                                          vol_center_pos, dpr, dcn, pr)
        out.update(dpos3d_radii=dpr, dconics=dcn, dintensities=dI, dpos3d=dpos, dscale3d=dscale,
                   dquat=dquat)
    return out
