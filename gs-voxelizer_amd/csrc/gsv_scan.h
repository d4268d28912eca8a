// gsv_scan.h — int32 exclusive/inclusive prefix sums for gfx950 whose element
// loads and result stores are functors, so a producer's arithmetic (e.g.
// buckets per tile) and a consumer's scatter (e.g. bucket -> tile) ride along
// with the scan instead of needing launches of their own.
//
// Blocks of 256 threads x 8 items (2048 elements).  Two launches when there
// are at most 2048 blocks: block sums, then an apply pass in which every block
// adds up its predecessors' sums itself (<= 8 loads per thread).  Above that a
// third launch scans the block sums in one workgroup first.  Every pass is
// HBM-bound: 4 B read per element twice, plus the stores.
#pragma once

#include "gsv_device.h"

namespace gsv {
// unnamed: each translation unit that scans gets its own copies of the kernels
namespace {
namespace scan_detail {

constexpr int kThreads = 256;
constexpr int kItems = 8;
constexpr int kTile = kThreads * kItems;
constexpr int64_t kDirectBlocks = 2048;

// Inclusive scan of one int per lane across a 64-wide wave.
__device__ __forceinline__ int wave_inclusive(int v) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int o = __shfl_up(v, d, kWave);
        if (lane >= d) v += o;
    }
    return v;
}

// Exclusive scan of one int per thread over the block; *total gets the sum.
__device__ __forceinline__ int block_exclusive(int v, int *lds_waves, int *total) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int inc = wave_inclusive(v);
    if (lane == kWave - 1) lds_waves[wave] = inc;
    __syncthreads();
    int off = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) {
        const int t = lds_waves[w];
        off += (w < wave) ? t : 0;
        sum += t;
    }
    *total = sum;
    return off + inc - v;
}

// Block b's sum of ld(b * kTile .. (b + 1) * kTile) into part[b] (a workgroup
// of kThreads; lds_waves holds kThreads / kWave ints).
template <class Load>
__device__ __forceinline__ void block_sums_body(Load ld, int64_t n, int32_t *part, int b,
                                                int *lds_waves) {
    const int64_t base = (int64_t)b * kTile + (int64_t)threadIdx.x * kItems;
    int s = 0;
#pragma unroll
    for (int k = 0; k < kItems; ++k)
        if (base + k < n) s += ld(base + k);
    int total;
    (void)block_exclusive(s, lds_waves, &total);
    if (threadIdx.x == 0) part[b] = total;
}
template <class Load>
__global__ __launch_bounds__(kThreads) void k_block_sums(Load ld, int64_t n, int32_t *part) {
    __shared__ int lds_waves[kThreads / kWave];
    block_sums_body(ld, n, part, (int)blockIdx.x, lds_waves);
}

// Writes the total to the device int64 and, when given, to pinned host memory
// (system-scope fence, so the host sees it once the kernel has completed).
__device__ __forceinline__ void put_total(int64_t v, int64_t *total_out, int64_t *total_host) {
    if (total_out) *total_out = v;
    if (total_host) {
        *reinterpret_cast<volatile int64_t *>(total_host) = v;
        __threadfence_system();
    }
}

// Exclusive scan of part[0..nb) in place by one workgroup of kSumsThreads;
// writes the total (int64: a sum beyond int32 stays visible to the caller).
// Tiles of kSumsThreads * 8: thread t loads 8 consecutive values (two 16-byte
// loads when part is 16-byte aligned), one block scan gives the offsets, and
// the prefixes are stored the same way, so every access is coalesced.
constexpr int kSumsThreads = 1024;

__global__ __launch_bounds__(kSumsThreads) void k_scan_block_sums(int32_t *part, int64_t nb,
                                                                  int64_t *total_out,
                                                                  int64_t *total_host) {
    __shared__ long long lds_waves[kSumsThreads / kWave];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const bool vec = (reinterpret_cast<uintptr_t>(part) & 15) == 0;
    long long carry = 0;
    for (int64_t base = 0; base < nb; base += (int64_t)kSumsThreads * kItems) {
        const int64_t i0 = base + (int64_t)threadIdx.x * kItems;
        const bool whole = vec && i0 + kItems <= nb;
        int v[kItems];
        if (whole) {
            const int4 a = *reinterpret_cast<const int4 *>(part + i0);
            const int4 b = *reinterpret_cast<const int4 *>(part + i0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int k = 0; k < kItems; ++k) v[k] = i0 + k < nb ? part[i0 + k] : 0;
        }
        long long s = 0;
#pragma unroll
        for (int k = 0; k < kItems; ++k) s += v[k];
        long long inc = s;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const long long o = __shfl_up(inc, d, kWave);
            if (lane >= d) inc += o;
        }
        if (lane == kWave - 1) lds_waves[wave] = inc;
        __syncthreads();
        long long run = carry + inc - s, total = 0;
#pragma unroll
        for (int w = 0; w < kSumsThreads / kWave; ++w) {
            const long long x = lds_waves[w];
            run += w < wave ? x : 0;
            total += x;
        }
        int o[kItems];
#pragma unroll
        for (int k = 0; k < kItems; ++k) {
            o[k] = (int32_t)run;
            run += v[k];
        }
        if (whole) {
            *reinterpret_cast<int4 *>(part + i0) = make_int4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<int4 *>(part + i0 + 4) = make_int4(o[4], o[5], o[6], o[7]);
        } else {
#pragma unroll
            for (int k = 0; k < kItems; ++k)
                if (i0 + k < nb) part[i0 + k] = o[k];
        }
        carry += total;
        __syncthreads();  // lds_waves is rewritten by the next tile
    }
    if (threadIdx.x == 0) put_total(carry, total_out, total_host);
}

// st(i, exclusive prefix of element i, element i) for every i < n.  direct:
// part holds raw block sums and each block adds its predecessors' (the last
// block then writes the total); otherwise part is already scanned.
// Block b of nblocks (a workgroup of kThreads; LDS as k_apply declares it).
template <class Load, class Store>
__device__ __forceinline__ void apply_body(Load ld, Store st, int64_t n, const int32_t *part,
                                           int direct, int64_t *total_out, int64_t *total_host,
                                           int b, int nblocks, int *lds_waves,
                                           long long *lds_pre) {
    long long prefix;
    if (direct) {
        long long s = 0;
        for (int j = threadIdx.x; j < b; j += kThreads) s += part[j];
#pragma unroll
        for (int o = kWave / 2; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
        if ((threadIdx.x & (kWave - 1)) == 0) lds_pre[threadIdx.x / kWave] = s;
        __syncthreads();
        prefix = 0;
#pragma unroll
        for (int w = 0; w < kThreads / kWave; ++w) prefix += lds_pre[w];
    } else {
        prefix = part[b];
    }
    const int64_t base = (int64_t)b * kTile + (int64_t)threadIdx.x * kItems;
    int v[kItems];
    int s = 0;
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        v[k] = (base + k < n) ? ld(base + k) : 0;
        s += v[k];
    }
    int total;
    int run = (int)(block_exclusive(s, lds_waves, &total) + prefix);
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        if (base + k < n) st(base + k, run, v[k]);
        run += v[k];
    }
    if (direct && b == nblocks - 1 && threadIdx.x == 0)
        put_total(prefix + total, total_out, total_host);
}
template <class Load, class Store>
__global__ __launch_bounds__(kThreads) void k_apply(Load ld, Store st, int64_t n,
                                                    const int32_t *part, int direct,
                                                    int64_t *total_out, int64_t *total_host) {
    __shared__ int lds_waves[kThreads / kWave];
    __shared__ long long lds_pre[kThreads / kWave];
    apply_body(ld, st, n, part, direct, total_out, total_host, (int)blockIdx.x, (int)gridDim.x,
               lds_waves, lds_pre);
}

}  // namespace scan_detail
}  // namespace

// Workspace of scan_run for n elements (the block sums).
inline size_t scan_workspace_bytes(int64_t n) {
    const int64_t nb = (n + scan_detail::kTile - 1) / scan_detail::kTile;
    return (size_t)((nb + 64) * sizeof(int32_t) + 255) / 256 * 256;
}

// Prefix sum of ld(0..n) handed to st; *total_out (optional, device int64)
// and *total_host (optional, device-visible pinned host int64) receive the sum.
// Launches on `stream`; no host synchronisation.
template <class Load, class Store>
int scan_run(Load ld, Store st, int64_t n, int64_t *total_out, int64_t *total_host, void *ws,
             size_t ws_bytes, hipStream_t stream) {
    using namespace scan_detail;
    if (n < 0) return GSV_ERR_INVALID_ARGUMENT;
    if (ws_bytes < scan_workspace_bytes(n) || !ws) return GSV_ERR_WORKSPACE_TOO_SMALL;
    const int64_t nb = (n + kTile - 1) / kTile;
    int32_t *part = static_cast<int32_t *>(ws);
    if (nb == 0) {
        hipLaunchKernelGGL(k_scan_block_sums, dim3(1), dim3(kSumsThreads), 0, stream, part, nb,
                           total_out, total_host);
        return check_launch();
    }
    hipLaunchKernelGGL(k_block_sums<Load>, dim3((unsigned)nb), dim3(kThreads), 0, stream, ld, n,
                       part);
    if (int st_ = check_launch()) return st_;
    const int direct = nb <= kDirectBlocks ? 1 : 0;
    if (!direct) {
        hipLaunchKernelGGL(k_scan_block_sums, dim3(1), dim3(kSumsThreads), 0, stream, part, nb,
                           total_out, total_host);
        if (int st_ = check_launch()) return st_;
    }
    hipLaunchKernelGGL((k_apply<Load, Store>), dim3((unsigned)nb), dim3(kThreads), 0, stream, ld,
                       st, n, part, direct, total_out, total_host);
    return check_launch();
}

struct LoadI32 {
    const int32_t *p;
    __device__ int operator()(int64_t i) const { return p[i]; }
};

struct StoreI32 {
    int32_t *out;
    int inclusive;
    __device__ void operator()(int64_t i, int excl, int v) const { out[i] = inclusive ? excl + v : excl; }
};

}  // namespace gsv
