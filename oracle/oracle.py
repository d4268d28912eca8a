"""numpy front-end of the C oracle. Test infrastructure only.

Two builds of ``gsv_oracle.c`` are wrapped:

* ``liboracle.so`` — binary32, the reference's arithmetic in its evaluation
  order; the module-level functions below use it;
* ``liboracle64.so`` — the same source in binary64 (``f64.<function>``, same
  signatures, float64 arrays), an estimate of each output's exact value for
  binary32 inputs.  The tests measure binary32 evaluations, this oracle's and
  the device's, against it.

Every function takes and returns contiguous numpy arrays with the layouts of the
reference API: pos3d/scale3d (N,3), quat (N,4) [w,x,y,z], intensities (N,C),
volume tuples (z, y, x), pos3d_radii (N,4), conics (N,6), tile_min/tile_max
(N,3) i32, num_tiles_hit (N,) i32, gaussian_ids_sorted (I,) i32, tile_bins
(T,2) i32, volume (D,H,W,C).  Float arrays are float32 for the binary32 build
and float64 for the binary64 one (inputs are converted).
"""
import ctypes
import os
import subprocess

import numpy as np

__all__ = [
    "lib", "build", "num_threads", "logf", "f2i_sat", "project_fwd", "project_bwd",
    "cumsum", "bin_and_sort", "voxelize_fwd", "voxelize_bwd", "tile_grid", "pipeline", "f64",
    "Oracle",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_c_int, _c_float, _c_i64 = ctypes.c_int, ctypes.c_float, ctypes.c_int64


def build():
    """Compile gsv_oracle.c into liboracle.so and liboracle64.so (gcc, no GPU needed)."""
    subprocess.check_call(["sh", os.path.join(_HERE, "build_oracle.sh")])


def tile_grid(vol_size_voxel):
    """(Tx, Ty, Tz) for a (D, H, W) volume, bindings.cu:70-74."""
    D, H, W = (int(v) for v in vol_size_voxel)
    return (W + 7) // 8, (H + 7) // 8, (D + 7) // 8


def _check(rc, name):
    if rc != 0:
        raise RuntimeError(f"oracle {name} failed with status {rc}")


def _i32(a, cols=None):
    a = np.ascontiguousarray(a, dtype=np.int32)
    if cols is not None:
        a = a.reshape(-1, cols)
    return a


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class Oracle:
    """One build of gsv_oracle.c: ``real`` is its float type (np.float32 or np.float64)."""

    def __init__(self, so_name, real):
        self.path = os.path.join(_HERE, so_name)
        self.real = np.dtype(real)
        self._lib = None

    def lib(self):
        if self._lib is None:
            if not os.path.exists(self.path):
                build()
            L = ctypes.CDLL(self.path)
            rp = np.ctypeslib.ndpointer(dtype=self.real, flags="C_CONTIGUOUS")
            rs = ctypes.c_double if self.real == np.float64 else ctypes.c_float
            L.orc_project_fwd.argtypes = [_c_int, _c_int, rp, rp, rp, rp, _c_int, _c_int, _c_int,
                                          rs, rs, rs, rs, rs, rs, rp, rp, _i32p, _i32p, _i32p]
            L.orc_project_bwd.argtypes = [_c_int, rp, rp, rp, _c_int, _c_int, _c_int,
                                          rs, rs, rs, rs, rs, rs, rp, rp, rp, rp, rp, rp]
            L.orc_cumsum_i32.argtypes = [_c_int, _i32p, _i32p]
            L.orc_cumsum_i32.restype = None
            L.orc_bin_and_sort.argtypes = [_c_int, _c_i64, _i32p, _i32p, _i32p, _c_int, _c_int,
                                           _c_int, _i32p, _i32p, ctypes.c_void_p]
            L.orc_voxelize_fwd.argtypes = [_c_int, _c_int, _c_int, _c_int, _i32p, _i32p, rp, rp,
                                           rp, rp, ctypes.c_void_p, _c_i64, _c_i64, _c_int,
                                           _c_int]
            L.orc_voxelize_bwd.argtypes = [_c_int, _c_int, _c_int, _c_int, _c_int, _i32p, _i32p,
                                           rp, rp, rp, rp, rp, rp, rp] + \
                [ctypes.c_void_p] * 6 + [_c_i64, _c_i64]
            L.orc_logf.argtypes = [_c_float]
            L.orc_logf.restype = _c_float
            L.orc_f2i_sat.argtypes = [_c_float]
            L.orc_f2i_sat.restype = _c_int
            L.orc_num_threads.restype = _c_int
            self._lib = L
        return self._lib

    def _r(self, a, cols=None):
        a = np.ascontiguousarray(a, dtype=self.real)
        if cols is not None:
            a = a.reshape(-1, cols)
        return a

    def num_threads(self):
        return self.lib().orc_num_threads()

    def project_fwd(self, pos3d, scale3d, quat, intensities, vol_size_voxel, vol_size_world,
                    vol_center_pos):
        pos3d, scale3d, quat = self._r(pos3d, 3), self._r(scale3d, 3), self._r(quat, 4)
        n = pos3d.shape[0]
        intensities = self._r(intensities).reshape(n, -1)
        C = intensities.shape[1]
        D, H, W = (int(v) for v in vol_size_voxel)
        wz, wy, wx = (float(v) for v in vol_size_world)
        cz, cy, cx = (float(v) for v in vol_center_pos)
        pr = np.empty((n, 4), self.real)
        cn = np.empty((n, 6), self.real)
        tmin = np.empty((n, 3), np.int32)
        tmax = np.empty((n, 3), np.int32)
        nt = np.empty((n,), np.int32)
        _check(self.lib().orc_project_fwd(n, C, pos3d, scale3d, quat, intensities, D, H, W, wz,
                                          wy, wx, cz, cy, cx, pr, cn, tmin, tmax, nt),
               "project_fwd")
        return pr, cn, tmin, tmax, nt

    def project_bwd(self, pos3d, scale3d, quat, vol_size_voxel, vol_size_world, vol_center_pos,
                    dpos_radii, dconics, pos_radii):
        pos3d, scale3d, quat = self._r(pos3d, 3), self._r(scale3d, 3), self._r(quat, 4)
        n = pos3d.shape[0]
        D, H, W = (int(v) for v in vol_size_voxel)
        wz, wy, wx = (float(v) for v in vol_size_world)
        cz, cy, cx = (float(v) for v in vol_center_pos)
        dp = np.empty((n, 3), self.real)
        ds = np.empty((n, 3), self.real)
        dq = np.empty((n, 4), self.real)
        _check(self.lib().orc_project_bwd(n, pos3d, scale3d, quat, D, H, W, wz, wy, wx, cz, cy,
                                          cx, self._r(dpos_radii, 4), self._r(dconics, 6),
                                          self._r(pos_radii, 4), dp, ds, dq), "project_bwd")
        return dp, ds, dq

    def cumsum(self, num_tiles_hit):
        x = _i32(num_tiles_hit).reshape(-1)
        out = np.empty_like(x)
        self.lib().orc_cumsum_i32(x.shape[0], x, out)
        return out

    def bin_and_sort(self, num_gaussians, num_intersects, tile_min, tile_max, cum_tiles_hit,
                     vol_size, return_keys=False):
        tmin, tmax = _i32(tile_min, 3), _i32(tile_max, 3)
        cum = _i32(cum_tiles_hit).reshape(-1)
        D, H, W = (int(v) for v in vol_size)
        Tx, Ty, Tz = tile_grid(vol_size)
        T = Tx * Ty * Tz
        I = max(int(num_intersects), 0)
        ids = np.empty((I,), np.int32)
        bins = np.empty((T, 2), np.int32)
        keys = np.empty((I,), np.int32) if return_keys else None
        _check(self.lib().orc_bin_and_sort(int(num_gaussians), int(num_intersects), tmin, tmax,
                                           cum, D, H, W, ids, bins,
                                           _ptr(keys) if return_keys else None),
               "bin_and_sort")
        return (ids, bins, keys) if return_keys else (ids, bins)

    def voxelize_fwd(self, vol_size, ids_sorted, tile_bins, pos_radii, conics, intensities,
                     tile_range=None, with_amb=False, z_slab=None):
        """(D,H,W,C) volume; with ``with_amb`` also the per-voxel sum of |I*alpha|
        over gate-ambiguous evaluations (see gate_ambiguous in gsv_oracle.c).
        With ``z_slab = (z0, z1)`` only the voxel planes [z0, z1) are held and
        returned, (z1 - z0, H, W, C) (pair it with a tile_range inside them)."""
        D, H, W = (int(v) for v in vol_size)
        z0, z1 = (0, D) if z_slab is None else (int(z_slab[0]), int(z_slab[1]))
        pr = self._r(pos_radii, 4)
        n = pr.shape[0]
        I = self._r(intensities).reshape(n, -1)
        C = I.shape[1]
        out = np.zeros((z1 - z0, H, W, C), self.real)
        amb = np.zeros((z1 - z0, H, W, C), self.real) if with_amb else None
        bins = _i32(tile_bins, 2)
        t0, t1 = tile_range if tile_range is not None else (0, bins.shape[0])
        _check(self.lib().orc_voxelize_fwd(D, H, W, C, _i32(ids_sorted).reshape(-1), bins, pr,
                                           self._r(conics, 6), I, out,
                                           _ptr(amb) if with_amb else None, int(t0), int(t1),
                                           z0, z1 - z0),
               "voxelize_fwd")
        return (out, amb) if with_amb else out

    def voxelize_bwd(self, vol_size, ids_sorted, tile_bins, pos_radii, conics, intensities,
                     vol_grad, tile_range=None, diagnostics=False):
        """Returns (dpos_radii (N,4), dconics (N,6), dintens (N,C)).  With
        ``diagnostics`` returns (grads, abs_sums, ambiguous_sums), each a triple in
        the same layout: per element the sum of |term| over contributing voxels
        (conditioning) and over gate-ambiguous evaluations."""
        D, H, W = (int(v) for v in vol_size)
        pr = self._r(pos_radii, 4)
        n = pr.shape[0]
        I = self._r(intensities).reshape(n, -1)
        C = I.shape[1]
        g = self._r(vol_grad).reshape(D, H, W, C)
        bins = _i32(tile_bins, 2)
        t0, t1 = tile_range if tile_range is not None else (0, bins.shape[0])
        trip = lambda: (np.empty((n, 4), self.real), np.empty((n, 6), self.real),
                        np.empty((n, C), self.real))
        grads = trip()
        absum, amb = (trip(), trip()) if diagnostics else (None, None)
        extra = ([_ptr(a) for a in absum] + [_ptr(a) for a in amb]) if diagnostics else [None] * 6
        _check(self.lib().orc_voxelize_bwd(D, H, W, C, n, _i32(ids_sorted).reshape(-1), bins, pr,
                                           self._r(conics, 6), I, g, grads[0], grads[1],
                                           grads[2], *extra, int(t0), int(t1)), "voxelize_bwd")
        return (grads, absum, amb) if diagnostics else grads

    def pipeline(self, pos3d, scale3d, quat, intensities, vol_size_voxel, vol_size_world,
                 vol_center_pos, vol_grad=None):
        """Whole forward (and, given vol_grad, backward) on the CPU, as the
        reference's Python layer sequences it (optim_to_render.py:56-149,
        voxelize.py:55-173). Returns a dict of every intermediate."""
        pr, cn, tmin, tmax, nt = self.project_fwd(pos3d, scale3d, quat, intensities,
                                                  vol_size_voxel, vol_size_world, vol_center_pos)
        n = pr.shape[0]
        I = self._r(intensities).reshape(n, -1)
        cum = self.cumsum(nt)
        n_isect = int(cum[-1]) if n > 0 else 0
        ids, bins = self.bin_and_sort(n, n_isect, tmin, tmax, cum, vol_size_voxel)
        vol = self.voxelize_fwd(vol_size_voxel, ids, bins, pr, cn, I)
        out = dict(pos3d_radii=pr, conics=cn, tile_min=tmin, tile_max=tmax, num_tiles_hit=nt,
                   cum_tiles_hit=cum, num_intersects=n_isect, gaussian_ids_sorted=ids,
                   tile_bins=bins, volume=vol)
        if vol_grad is not None:
            dpr, dcn, dI = self.voxelize_bwd(vol_size_voxel, ids, bins, pr, cn, I, vol_grad)
            dpos, dscale, dquat = self.project_bwd(pos3d, scale3d, quat, vol_size_voxel,
                                                   vol_size_world, vol_center_pos, dpr, dcn, pr)
            out.update(dpos3d_radii=dpr, dconics=dcn, dintensities=dI, dpos3d=dpos,
                       dscale3d=dscale, dquat=dquat)
        return out


_f32 = Oracle("liboracle.so", np.float32)
f64 = Oracle("liboracle64.so", np.float64)

lib = _f32.lib
num_threads = _f32.num_threads
project_fwd = _f32.project_fwd
project_bwd = _f32.project_bwd
cumsum = _f32.cumsum
bin_and_sort = _f32.bin_and_sort
voxelize_fwd = _f32.voxelize_fwd
voxelize_bwd = _f32.voxelize_bwd
pipeline = _f32.pipeline


def logf(x):
    return lib().orc_logf(float(x))


def f2i_sat(x):
    return lib().orc_f2i_sat(float(x))
