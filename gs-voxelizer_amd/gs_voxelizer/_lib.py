"""Loader for libgsvox.so, the gfx950 C-ABI library (declared in include/gsvox.h).

There is no fallback: if the library is missing or does not load, importing
``gs_voxelizer.cuda`` raises, exactly as the reference's import of its CUDA
extension does (optim_to_render.py:10, voxelize.py:9).
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.environ.get("GSV_LIBRARY", os.path.join(_HERE, "libgsvox.so"))

_c_int, _c_i64, _c_float, _c_void_p, _c_size_t = (ctypes.c_int32, ctypes.c_int64, ctypes.c_float,
                                                   ctypes.c_void_p, ctypes.c_size_t)
_P = _c_void_p

# name -> argument types, in the order of include/gsvox.h
SIGNATURES = {
    "gsv_version": [],
    "gsv_status_string": [_c_int],
    "gsv_last_hip_error": [],
    "gsv_project_fwd": [_c_int, _c_int, _P, _P, _P, _P, _c_int, _c_int, _c_int,
                        _c_float, _c_float, _c_float, _c_float, _c_float, _c_float,
                        _P, _P, _P, _P, _P, _P],
    "gsv_project_bwd": [_c_int, _P, _P, _P, _c_int, _c_int, _c_int,
                        _c_float, _c_float, _c_float, _c_float, _c_float, _c_float,
                        _P, _P, _P, _P, _P, _P, _P],
    "gsv_scan_workspace_bytes": [_c_i64, ctypes.POINTER(_c_size_t)],
    "gsv_cumsum_tiles_hit": [_c_int, _P, _P, _P, _P, _P, _c_size_t, _P],
    "gsv_bin_workspace_bytes": [_c_int, _c_i64, _c_int, _c_int, _c_int, ctypes.POINTER(_c_size_t)],
    "gsv_bin_and_sort": [_c_int, _c_i64, _P, _P, _P, _c_int, _c_int, _c_int, _P, _c_size_t,
                         _P, _P, _P, _P],
    "gsv_bin_and_sort_device_count": [_c_int, _c_i64, _P, _P, _P, _P, _c_int, _c_int, _c_int, _P,
                                      _c_size_t, _P, _P, _P, _P],
    "gsv_cumsum_bin_workspace_bytes": [_c_int, _c_i64, _c_int, _c_int, _c_int,
                                       ctypes.POINTER(_c_size_t)],
    "gsv_cumsum_bin_and_sort_device_count": [_c_int, _c_i64, _P, _P, _P, _c_int, _c_int, _c_int,
                                             _P, _P, _P, _P, _c_size_t, _P, _P, _P, _P],
    "gsv_bin_and_sort_noalloc": [_c_int, _c_i64, _P, _P, _P, _c_int, _c_int, _c_int, _P, _P, _P,
                                 _P],
    "gsv_voxelize_fwd": [_c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _P, _P, _P, _P, _P, _P,
                         _P, _P],
    "gsv_set_backward_chains": [_c_int, ctypes.POINTER(_c_int)],
    "gsv_voxelize_fwd_l1_workspace_bytes": [_c_int, _c_int, _c_int, ctypes.POINTER(_c_size_t)],
    "gsv_voxelize_fwd_l1": [_c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _P, _P, _P, _P, _P,
                            _P, _P, _P, _P, _P, _P, _c_size_t, _P],
    "gsv_voxelize_bwd_workspace_bytes": [_c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int,
                                         ctypes.POINTER(_c_size_t)],
    "gsv_voxelize_bwd": [_c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _P, _P, _P, _P, _P, _P,
                         _P, _P, _P, _P, _P, _P, _P, _P, _P, _c_int, _P, _c_size_t, _P],
    "gsv_voxelize_bwd_l1": [_c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _P, _P, _P, _P, _P,
                            _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _c_int, _P,
                            _c_size_t, _P],
    "gsv_kernel_timing_enable": [_c_int],
    "gsv_kernel_timing_collect": [_c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_int)],
    "gsv_wave_timeline": [_c_int, _P, _c_int],
}

_lib = None


def load():
    """Load (once) and return the ctypes handle; raises OSError if unavailable."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise OSError(
                f"gs_voxelizer: native library not found at {LIBRARY_PATH}. Build it with "
                "`python gs-voxelizer_amd/build.py` (hipcc, --offload-arch=gfx950).")
        lib = ctypes.CDLL(LIBRARY_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_char_p if name == "gsv_status_string" else ctypes.c_int
        _lib = lib
    return _lib
