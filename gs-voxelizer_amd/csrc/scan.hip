// scan.hip — int32 prefix sums (reduce-then-scan), zero fill, status glue.
//
// Used for the per-Gaussian tile counts (the reference's torch.cumsum,
// voxelize.py:87), for the radix-sort digit histograms and for the backward's
// bucket offsets.  Three launches: block partial sums, an exclusive scan of the
// partials in one workgroup, and a block scan that adds each block's offset.
// Every pass is HBM-bound: 4 B read + 4 B written per element, plus 4 B read in
// the reduce pass.
#include <mutex>
#include <vector>

#include "gsv_device.h"

namespace gsv {

namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;  // 2048 elements per block

thread_local int t_last_hip_error = 0;

// Inclusive scan of one int per lane across a 64-wide wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int o = __shfl_up(v, d, kWave);
        if (lane >= d) v += o;
    }
    return v;
}

// Exclusive scan of one int per thread over a 256-thread block; returns the
// exclusive prefix and writes the block total to *total.
__device__ __forceinline__ int block_exclusive_scan(int v, int *lds_waves, int *total) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int inc = wave_inclusive_scan(v);
    if (lane == kWave - 1) lds_waves[wave] = inc;
    __syncthreads();
    int off = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / kWave; ++w) {
        const int t = lds_waves[w];
        off += (w < wave) ? t : 0;
        sum += t;
    }
    *total = sum;
    return off + inc - v;
}

__global__ __launch_bounds__(kScanThreads) void k_scan_reduce(const int32_t *__restrict__ in,
                                                              int64_t n, int32_t *__restrict__ part) {
    __shared__ int lds_waves[kScanThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int s = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k)
        if (base + k < n) s += in[base + k];
    int total;
    (void)block_exclusive_scan(s, lds_waves, &total);
    if (threadIdx.x == 0) part[blockIdx.x] = total;
}

// Exclusive scan of part[0..nb) in place by one workgroup; optional int64 total.
__global__ __launch_bounds__(kScanThreads) void k_scan_partials(int32_t *__restrict__ part,
                                                                int64_t nb,
                                                                int64_t *__restrict__ total_out) {
    __shared__ int lds_waves[kScanThreads / kWave];
    int64_t carry = 0;
    for (int64_t start = 0; start < nb; start += kScanThreads) {
        const int64_t i = start + threadIdx.x;
        const int v = i < nb ? part[i] : 0;
        int total;
        const int ex = block_exclusive_scan(v, lds_waves, &total);
        if (i < nb) part[i] = (int32_t)(carry + ex);
        carry += total;
        __syncthreads();  // lds_waves reused by the next chunk
    }
    if (total_out && threadIdx.x == 0) *total_out = carry;
}

__global__ __launch_bounds__(kScanThreads) void k_scan_apply(const int32_t *__restrict__ in,
                                                             int32_t *__restrict__ out, int64_t n,
                                                             const int32_t *__restrict__ part,
                                                             int inclusive) {
    __shared__ int lds_waves[kScanThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int v[kScanItems];
    int s = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        v[k] = (base + k < n) ? in[base + k] : 0;
        s += v[k];
    }
    int total;
    int run = block_exclusive_scan(s, lds_waves, &total) + part[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int next = run + v[k];
        if (base + k < n) out[base + k] = inclusive ? next : run;
        run = next;
    }
}

__global__ __launch_bounds__(256) void k_fill_zero(uint32_t *__restrict__ p, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

}  // namespace

namespace {
struct TimingState {
    std::mutex mu;
    bool enabled = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending[kTimedCount];
    double total_ms[kTimedCount] = {0, 0, 0};
    int count[kTimedCount] = {0, 0, 0};
};
TimingState &timing() {
    static TimingState st;
    return st;
}
}  // namespace

KernelTimer::KernelTimer(int s, hipStream_t st) : slot(s), stream(st), stop(nullptr), on(false) {
    TimingState &T = timing();
    std::lock_guard<std::mutex> lk(T.mu);
    if (!T.enabled) return;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess) return;
    if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        return;
    }
    (void)hipEventRecord(a, stream);
    T.pending[slot].push_back({a, b});
    stop = b;
    on = true;
}

// The stop event is recorded right after the launch.  gsv_kernel_timing_collect
// must be called after the launches it measures have been issued.
KernelTimer::~KernelTimer() {
    if (on) (void)hipEventRecord(stop, stream);
}

int record_hip_error(hipError_t e) {
    t_last_hip_error = (int)e;
    return GSV_ERR_HIP;
}

int fill_zero_u32(void *ptr, int64_t n_words, hipStream_t stream) {
    if (n_words <= 0) return GSV_OK;
    int64_t blocks = (n_words + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<uint32_t *>(ptr), n_words);
    return check_launch();
}

size_t scan_workspace_bytes(int64_t n) {
    const int64_t nb = (n + kScanTile - 1) / kScanTile;
    return (size_t)((nb + 64) * sizeof(int32_t) + 255) / 256 * 256;
}

int scan_i32(const int32_t *in, int32_t *out, int64_t n, bool inclusive, int64_t *total_out,
             void *ws, size_t ws_bytes, hipStream_t stream) {
    if (n < 0) return GSV_ERR_INVALID_ARGUMENT;
    if (ws_bytes < scan_workspace_bytes(n) || (n > 0 && !ws)) return GSV_ERR_WORKSPACE_TOO_SMALL;
    const int64_t nb = (n + kScanTile - 1) / kScanTile;
    int32_t *part = static_cast<int32_t *>(ws);
    if (n > 0) {
        hipLaunchKernelGGL(k_scan_reduce, dim3((unsigned)nb), dim3(kScanThreads), 0, stream, in, n, part);
        if (int st = check_launch()) return st;
    }
    hipLaunchKernelGGL(k_scan_partials, dim3(1), dim3(kScanThreads), 0, stream, part, nb, total_out);
    if (int st = check_launch()) return st;
    if (n > 0) {
        hipLaunchKernelGGL(k_scan_apply, dim3((unsigned)nb), dim3(kScanThreads), 0, stream, in, out,
                           n, part, inclusive ? 1 : 0);
        if (int st = check_launch()) return st;
    }
    return GSV_OK;
}

}  // namespace gsv

using namespace gsv;

extern "C" int gsv_version(void) { return 100; }

extern "C" const char *gsv_status_string(int status) {
    switch (status) {
        case GSV_OK: return "ok";
        case GSV_ERR_INVALID_ARGUMENT: return "invalid argument";
        case GSV_ERR_UNSUPPORTED_CHANNELS: return "Number of channels exceeds MAX_CHANNELS (1..4 supported)";
        case GSV_ERR_WORKSPACE_TOO_SMALL: return "workspace too small";
        case GSV_ERR_SIZE_OVERFLOW: return "size exceeds the int32 index range";
        case GSV_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

extern "C" int gsv_last_hip_error(void) { return t_last_hip_error; }

extern "C" int gsv_kernel_timing_enable(int32_t enable) {
    TimingState &T = timing();
    std::lock_guard<std::mutex> lk(T.mu);
    T.enabled = enable != 0;
    return GSV_OK;
}

extern "C" int gsv_kernel_timing_collect(int32_t kernel, double *total_ms, int32_t *count) {
    if (kernel < 0 || kernel >= kTimedCount || !total_ms || !count) return GSV_ERR_INVALID_ARGUMENT;
    TimingState &T = timing();
    std::lock_guard<std::mutex> lk(T.mu);
    for (auto &ev : T.pending[kernel]) {
        float ms = 0.f;
        hipError_t e = hipEventSynchronize(ev.second);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.first, ev.second);
        (void)hipEventDestroy(ev.first);
        (void)hipEventDestroy(ev.second);
        if (e != hipSuccess) {
            T.pending[kernel].clear();
            return record_hip_error(e);
        }
        T.total_ms[kernel] += ms;
        T.count[kernel] += 1;
    }
    T.pending[kernel].clear();
    *total_ms = T.total_ms[kernel];
    *count = T.count[kernel];
    T.total_ms[kernel] = 0;
    T.count[kernel] = 0;
    return GSV_OK;
}

extern "C" int gsv_scan_workspace_bytes(int64_t n, size_t *bytes) {
    if (n < 0 || !bytes) return GSV_ERR_INVALID_ARGUMENT;
    *bytes = scan_workspace_bytes(n);
    return GSV_OK;
}

extern "C" int gsv_cumsum_tiles_hit(int32_t n, const int32_t *num_tiles_hit,
                                    int32_t *cum_tiles_hit, int64_t *total_out, void *workspace,
                                    size_t workspace_bytes, void *stream) {
    if (n < 0) return GSV_ERR_INVALID_ARGUMENT;
    if (n > 0 && (!num_tiles_hit || !cum_tiles_hit)) return GSV_ERR_INVALID_ARGUMENT;
    return scan_i32(num_tiles_hit, cum_tiles_hit, n, true, total_out, workspace, workspace_bytes,
                    as_stream(stream));
}
