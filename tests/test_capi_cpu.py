"""The C-ABI library without a GPU: it loads, exports every entry point that
include/gsvox.h declares, and its host-side validation / sizing answers
without touching a device."""
import ctypes
import os
import re

import pytest

from gs_voxelizer import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "gsvox.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gsv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    names = _declared()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_status_strings_and_version():
    L = _lib.load()
    assert L.gsv_version() >= 100
    for code in range(7):
        assert L.gsv_status_string(code)
    assert b"MAX_CHANNELS" in L.gsv_status_string(2)
    assert L.gsv_status_string(99) == b"unknown status"


def test_validation_without_device():
    L = _lib.load()
    null = ctypes.c_void_p(0)
    # channels outside [1, 4] -> GSV_ERR_UNSUPPORTED_CHANNELS before any launch
    args = [10, 5] + [null] * 4 + [8, 8, 8] + [1.0] * 6 + [null] * 5 + [null]
    assert L.gsv_project_fwd(*args) == 2
    args[1] = 1
    args[0] = -1
    assert L.gsv_project_fwd(*args) == 1
    args[0] = 0  # empty input is a no-op
    assert L.gsv_project_fwd(*args) == 0
    assert L.gsv_voxelize_fwd(8, 8, 8, 0, 1, 1, *[null] * 7, null) == 2
    assert L.gsv_voxelize_bwd(8, 8, 8, 1, 1, 1, *[null] * 15, 7, null, 0, null) == 1


def test_workspace_sizes_are_host_only():
    L = _lib.load()
    b = ctypes.c_size_t(0)
    assert L.gsv_scan_workspace_bytes(1_000_000, ctypes.byref(b)) == 0 and b.value > 0
    assert L.gsv_bin_workspace_bytes(200_000, 3_542_885, 256, 256, 256, ctypes.byref(b)) == 0
    assert b.value >= 3 * 3_542_885 * 4
    small = b.value
    assert L.gsv_bin_workspace_bytes(200_000, 2**31, 256, 256, 256, ctypes.byref(b)) == 4
    assert L.gsv_voxelize_bwd_workspace_bytes(256, 256, 256, 1, 200_000, 3_542_885, 1,
                                              ctypes.byref(b)) == 0
    det = b.value
    assert L.gsv_voxelize_bwd_workspace_bytes(256, 256, 256, 1, 200_000, 3_542_885, 0,
                                              ctypes.byref(b)) == 0
    assert det - b.value >= 3_542_885 * 10 * 4  # per-pair partials of the deterministic mode
    assert b.value >= 200_000 * 128  # one 128-byte record per Gaussian
    assert L.gsv_voxelize_bwd_workspace_bytes(256, 256, 256, 1, -1, 3_542_885, 0,
                                              ctypes.byref(b)) == 1  # GSV_ERR_INVALID_ARGUMENT
    assert small > 0


def test_noalloc_binning_rejects_oversize_before_any_launch():
    """The allocation-free binning holds at most GSV_NOALLOC_MAX_INTERSECTIONS
    pairs; one more is refused on the host with its own status code."""
    L = _lib.load()
    null = ctypes.c_void_p(0)
    st = L.gsv_bin_and_sort_noalloc(10, 4194304 + 1, null, null, null, 256, 256, 256,
                                    null, null, null, null)
    assert st == 6
    assert b"allocation-free" in L.gsv_status_string(6)
    assert L.gsv_bin_and_sort_noalloc(-1, 10, null, null, null, 8, 8, 8,
                                      null, null, null, null) == 1


def test_wave_timeline_registration_is_host_only():
    L = _lib.load()
    null = ctypes.c_void_p(0)
    assert L.gsv_wave_timeline(1, null, 0) == 1       # only the forward kernel
    assert L.gsv_wave_timeline(0, null, -1) == 1
    assert L.gsv_wave_timeline(0, ctypes.c_void_p(256), 0) == 1
    assert L.gsv_wave_timeline(0, null, 0) == 0       # unregister
