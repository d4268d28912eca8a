// gsv_device.h — helpers shared by the gfx950 translation units of libgsvox.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gsvox.h"
#include "gsv_numerics.h"

namespace gsv {

// Records the failing hipError_t for gsv_last_hip_error() (thread-local).
int record_hip_error(hipError_t e);

// Returns GSV_OK or GSV_ERR_HIP after checking the last launch on this thread.
inline int check_launch() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? GSV_OK : record_hip_error(e);
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kWave = 64;    // CDNA wavefront width
constexpr int kXcds = 8;     // MI355X: 8 XCDs, each with its own L2

// Maps a launch-order block index to a work index so that consecutive work
// items land on the same XCD.  The hardware dispatches workgroup b to XCD
// (b mod 8); giving XCD k the contiguous range [k*per, (k+1)*per) keeps
// neighbouring tiles (which share Gaussians) in one L2.  Launch 8*per blocks;
// indices >= count must exit.
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t per) {
    return (b % kXcds) * per + b / kXcds;
}
__host__ __device__ inline int64_t xcd_per(int64_t count) { return (count + kXcds - 1) / kXcds; }

// Tile order for per-tile launches: runs of 8 consecutive tiles (along x)
// rotate over the XCDs, one run per XCD in each super-run S of 64 tiles, by
// S + S/8 + S/64 (the higher terms keep rows whose super-run index is a
// multiple of 8 from landing on the same XCDs).  Every XCD so gets an even
// share of every region of the volume (clustered scenes and the volume's faces
// included) while the tiles of a run share one L2.  Block b (dispatched to
// XCD b % 8) takes the tile returned, which is below kRunSpan * ceil(T /
// kRunSpan) = the grid size.
constexpr int kRunSpan = 8 * kXcds;
__device__ __forceinline__ int64_t xcd_runs(int64_t b) {
    const int64_t k = b % kXcds, j = b / kXcds;
    const int64_t S = j / 8, t = j % 8;
    return S * kRunSpan + ((k + S + (S >> 3) + (S >> 6)) % kXcds) * 8 + t;
}
__host__ __device__ inline int64_t xcd_runs_grid(int64_t T) {
    return (T + kRunSpan - 1) / kRunSpan * kRunSpan;
}
// floor(x / d) for 0 <= x < 2^31 and 1 <= d < 2^31 as a multiply and a shift:
// with 2^(s-1) < d <= 2^s and m = floor(2^(31+s) / d) + 1 (below 2^32), the
// error m*d - 2^(31+s) lies in (0, d], so x * (m*d - 2^(31+s)) < 2^(31+s) and
// (x * m) >> (31 + s) is exact (Granlund and Montgomery, "Division by invariant
// integers using multiplication", 1994).
struct FastDiv {
    uint32_t m;
    int s;
};
inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.s = 0;
    while ((1u << f.s) < d) ++f.s;
    f.m = (uint32_t)(((uint64_t)1 << (31 + f.s)) / d + 1);
    return f;
}
__device__ __forceinline__ uint32_t fastdiv(uint32_t x, FastDiv f) {
    return (uint32_t)(((uint64_t)x * f.m) >> (31 + f.s));
}

__host__ __device__ inline int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }
__host__ __device__ inline int64_t imax64(int64_t a, int64_t b) { return a > b ? a : b; }

// Optional per-kernel timing (gsv_kernel_timing_*): when enabled, the hot
// kernels are bracketed by HIP events recorded on their launch stream.
struct KernelTimer {
    int slot;
    hipStream_t stream;
    hipEvent_t stop;
    bool on;
    KernelTimer(int slot, hipStream_t s);
    ~KernelTimer();
};
enum TimedKernel { kTimedVoxFwd = 0, kTimedVoxBwd = 1, kTimedPairReduce = 2, kTimedCount = 3 };

// The buffer registered with gsv_wave_timeline for the forward kernel (or
// nullptr) and its capacity in workgroups.
uint64_t *wave_timeline_buffer(int *capacity);

// Zero-fills n 32-bit words with a kernel (graph-capture safe, unlike memset).
int fill_zero_u32(void *ptr, int64_t n_words, hipStream_t stream);

// The device address of a pinned (device-visible) host int64, or nullptr for
// host == nullptr; GSV_ERR_INVALID_ARGUMENT for memory that is not pinned.
int pinned_int64_device_ptr(int64_t *host, int64_t **dev);

// Exclusive / inclusive int32 scan of a device array (scan.hip; the functor
// form and scan_workspace_bytes are in gsv_scan.h).
int scan_i32(const int32_t *in, int32_t *out, int64_t n, bool inclusive, int64_t *total_out,
             int64_t *total_host, void *ws, size_t ws_bytes, hipStream_t stream);

}  // namespace gsv
