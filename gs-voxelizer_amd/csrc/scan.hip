// scan.hip — the per-Gaussian tile-count prefix sum (the reference's
// torch.cumsum, voxelize.py:87) on the functor scan of gsv_scan.h, the
// graph-safe zero fill, kernel timing and status glue.
#include <mutex>
#include <vector>

#include "gsv_device.h"
#include "gsv_scan.h"

namespace gsv {

namespace {

thread_local int t_last_hip_error = 0;

__global__ __launch_bounds__(256) void k_fill_zero(uint32_t *__restrict__ p, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

}  // namespace

namespace {
// Event pairs are pooled: creating HIP events costs host time, and the timed
// launches sit inside the caller's measured loop.
struct TimingState {
    std::mutex mu;
    bool enabled = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pool;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending[kTimedCount];
    double total_ms[kTimedCount] = {0, 0, 0};
    int count[kTimedCount] = {0, 0, 0};
};
TimingState &timing() {
    static TimingState st;
    return st;
}
bool take_pair(TimingState &T, std::pair<hipEvent_t, hipEvent_t> *out) {
    if (!T.pool.empty()) {
        *out = T.pool.back();
        T.pool.pop_back();
        return true;
    }
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess) return false;
    if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        return false;
    }
    *out = {a, b};
    return true;
}
}  // namespace

KernelTimer::KernelTimer(int s, hipStream_t st) : slot(s), stream(st), stop(nullptr), on(false) {
    TimingState &T = timing();
    std::lock_guard<std::mutex> lk(T.mu);
    if (!T.enabled) return;
    std::pair<hipEvent_t, hipEvent_t> ev;
    if (!take_pair(T, &ev)) return;
    (void)hipEventRecord(ev.first, stream);
    T.pending[slot].push_back(ev);
    stop = ev.second;
    on = true;
}

// The stop event is recorded right after the launch.  gsv_kernel_timing_collect
// must be called after the launches it measures have been issued.
KernelTimer::~KernelTimer() {
    if (on) (void)hipEventRecord(stop, stream);
}

namespace {
std::mutex g_wave_mu;
uint64_t *g_wave_records = nullptr;
int g_wave_capacity = 0;
int g_wave_device = -1;  // the device current when the buffer was registered
}  // namespace

uint64_t *wave_timeline_buffer(int *capacity) {
    std::lock_guard<std::mutex> lk(g_wave_mu);
    int dev = -1;
    if (g_wave_records == nullptr || hipGetDevice(&dev) != hipSuccess || dev != g_wave_device) {
        *capacity = 0;
        return nullptr;  // none registered, or registered for another device
    }
    *capacity = g_wave_capacity;
    return g_wave_records;
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

int pinned_int64_device_ptr(int64_t *host, int64_t **dev) {
    *dev = nullptr;
    if (!host) return GSV_OK;
    void *p = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&p, host, 0);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // leave no error behind for the next launch check
        (void)record_hip_error(e);
        return GSV_ERR_INVALID_ARGUMENT;  // not pinned, device-visible host memory
    }
    *dev = static_cast<int64_t *>(p);
    return GSV_OK;
}

int scan_i32(const int32_t *in, int32_t *out, int64_t n, bool inclusive, int64_t *total_out,
             int64_t *total_host, void *ws, size_t ws_bytes, hipStream_t stream) {
    if (n > 0 && (!in || !out)) return GSV_ERR_INVALID_ARGUMENT;
    return scan_run(LoadI32{in}, StoreI32{out, inclusive ? 1 : 0}, n, total_out, total_host, ws,
                    ws_bytes, stream);
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
        case GSV_ERR_SCRATCH_TOO_SMALL:
            return "more intersections than the allocation-free binning's fixed scratch holds "
                   "(GSV_NOALLOC_MAX_INTERSECTIONS)";
        default: return "unknown status";
    }
}

extern "C" int gsv_last_hip_error(void) { return t_last_hip_error; }

extern "C" int gsv_kernel_timing_enable(int32_t enable) {
    TimingState &T = timing();
    std::lock_guard<std::mutex> lk(T.mu);
    T.enabled = enable != 0;
    // pre-create a pool so the first timed launches do not create events
    size_t have = T.pool.size();
    for (int k = 0; k < kTimedCount; ++k) have += T.pending[k].size();
    for (; T.enabled && have < 64; ++have) {
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess) break;
        if (hipEventCreate(&b) != hipSuccess) {
            (void)hipEventDestroy(a);
            break;
        }
        T.pool.push_back({a, b});
    }
    return GSV_OK;
}

extern "C" int gsv_kernel_timing_collect(int32_t kernel, double *total_ms, int32_t *count) {
    if (kernel < 0 || kernel >= kTimedCount || !total_ms || !count) return GSV_ERR_INVALID_ARGUMENT;
    TimingState &T = timing();
    std::lock_guard<std::mutex> lk(T.mu);
    hipError_t err = hipSuccess;
    for (auto &ev : T.pending[kernel]) {
        float ms = 0.f;
        hipError_t e = hipEventSynchronize(ev.second);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.first, ev.second);
        T.pool.push_back(ev);
        if (e != hipSuccess) {
            err = e;
            continue;
        }
        T.total_ms[kernel] += ms;
        T.count[kernel] += 1;
    }
    T.pending[kernel].clear();
    *total_ms = T.total_ms[kernel];
    *count = T.count[kernel];
    T.total_ms[kernel] = 0;
    T.count[kernel] = 0;
    return err == hipSuccess ? GSV_OK : record_hip_error(err);
}

extern "C" int gsv_scan_workspace_bytes(int64_t n, size_t *bytes) {
    if (n < 0 || !bytes) return GSV_ERR_INVALID_ARGUMENT;
    *bytes = scan_workspace_bytes(n);
    return GSV_OK;
}

extern "C" int gsv_cumsum_tiles_hit(int32_t n, const int32_t *num_tiles_hit,
                                    int32_t *cum_tiles_hit, int64_t *total_out,
                                    int64_t *total_host, void *workspace, size_t workspace_bytes,
                                    void *stream) {
    if (n < 0) return GSV_ERR_INVALID_ARGUMENT;
    if (n > 0 && (!num_tiles_hit || !cum_tiles_hit)) return GSV_ERR_INVALID_ARGUMENT;
    int64_t *host_dev = nullptr;  // the kernels' address of the pinned host int64
    if (int st = pinned_int64_device_ptr(total_host, &host_dev)) return st;
    return scan_i32(num_tiles_hit, cum_tiles_hit, n, true, total_out, host_dev, workspace,
                    workspace_bytes, as_stream(stream));
}

extern "C" int gsv_wave_timeline(int32_t kernel, uint64_t *records, int32_t capacity) {
    if (kernel != 0 || capacity < 0 || (records != nullptr && capacity == 0))
        return GSV_ERR_INVALID_ARGUMENT;
    int dev = -1;
    if (records != nullptr) {
        const hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return record_hip_error(e);
    }
    std::lock_guard<std::mutex> lk(g_wave_mu);
    g_wave_records = records;
    g_wave_capacity = records ? capacity : 0;
    g_wave_device = dev;
    return GSV_OK;
}
