// binning.hip — (tile, gaussian) key duplication, stable LSD radix sort over the
// significant tile-id bits, and tile-range extraction, for gfx950.
//
// Reference: gs_voxelizer/cuda/bin_and_sort_gaussians.cu:11-62 and the binding
// bindings.cu:259-360 (which sorts all 32 key bits with cub::DeviceRadixSort).
// Keys are tile ids < T, so only ceil(log2 T) bits are sorted here (15 at 256^3:
// two 8-bit passes instead of four).  Because the keys are emitted
// gaussian-major and every pass is stable, the result is the reference's exact
// order: ascending tile, then ascending gaussian id.
//
// Data movement per pair: emission writes 8 B; each radix pass reads 4 B
// (histogram) + 8 B and writes 8 B; the range pass reads 4 B.
#include "gsv_device.h"

namespace gsv {
namespace {

constexpr int kEmitThreads = 256;
constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;  // 4096 keys per block
constexpr int kRadixBits = 8;
constexpr int kRadixBins = 1 << kRadixBits;
static_assert(kRadixBins == kSortThreads, "one digit per thread in the block scans");

// One block emits the pairs of 256 consecutive Gaussians.  Their output ranges
// are contiguous ([cum[g-1], cum[g])), so the block walks its whole output range
// with coalesced stores and finds each slot's Gaussian by binary search in LDS,
// instead of one serial loop per Gaussian (which stalls on large Gaussians).
__global__ __launch_bounds__(kEmitThreads) void k_emit(
    int n, int64_t n_isect, const int *__restrict__ tile_min, const int *__restrict__ tile_max,
    const int *__restrict__ cum, int Tx, int Ty, int *__restrict__ keys, int *__restrict__ vals) {
    __shared__ int s_start[kEmitThreads];
    __shared__ int s_cnt[kEmitThreads];
    __shared__ int s_box[kEmitThreads][5];  // min x, y, z; extent x, y
    const int t = threadIdx.x;
    const int g0 = blockIdx.x * kEmitThreads;
    const int g = g0 + t;
    const int last = min(g0 + kEmitThreads, n) - 1;
    int start = 0, cnt = 0;
    if (g < n) {
        start = g == 0 ? 0 : cum[g - 1];
        const int mnx = tile_min[3 * g], mny = tile_min[3 * g + 1], mnz = tile_min[3 * g + 2];
        const int ex = tile_max[3 * g] - mnx, ey = tile_max[3 * g + 1] - mny,
                  ez = tile_max[3 * g + 2] - mnz;
        const int64_t box = (ex > 0 && ey > 0 && ez > 0) ? (int64_t)ex * ey * ez : 0;
        const int64_t avail = (int64_t)cum[g] - start;
        cnt = (int)max<int64_t>(0, min(box, avail));
        s_box[t][0] = mnx; s_box[t][1] = mny; s_box[t][2] = mnz;
        s_box[t][3] = max(ex, 1); s_box[t][4] = max(ey, 1);
    } else {
        start = 0x7fffffff;  // sorts after every real start
    }
    s_start[t] = start;
    s_cnt[t] = cnt;
    __syncthreads();
    const int64_t lo = max<int64_t>(0, s_start[0]);
    const int64_t hi = min<int64_t>(n_isect, (int64_t)cum[last]);
    for (int64_t p = lo + t; p < hi; p += kEmitThreads) {
        // largest l with s_start[l] <= p
        int l = 0;
#pragma unroll
        for (int step = kEmitThreads / 2; step > 0; step >>= 1)
            if (s_start[l + step] <= p) l += step;
        const int j = (int)(p - s_start[l]);
        if (j < 0 || j >= s_cnt[l]) continue;
        const int nx = s_box[l][3], ny = s_box[l][4];
        const int dx = j % nx, r = j / nx;
        const int dy = r % ny, dz = r / ny;
        keys[p] = (s_box[l][2] + dz) * Ty * Tx + (s_box[l][1] + dy) * Tx + (s_box[l][0] + dx);
        vals[p] = g0 + l;
    }
}

// Per-block digit histogram, stored digit-major: hist[d * nblocks + block].
__global__ __launch_bounds__(kSortThreads) void k_radix_hist(const int *__restrict__ keys,
                                                             int64_t n, int shift,
                                                             int *__restrict__ hist, int nblocks) {
    __shared__ int s_hist[kRadixBins];
    const int t = threadIdx.x;
    s_hist[t] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t i = base + (int64_t)k * kSortThreads + t;
        if (i < n) atomicAdd(&s_hist[(keys[i] >> shift) & (kRadixBins - 1)], 1);
    }
    __syncthreads();
    hist[(int64_t)t * nblocks + blockIdx.x] = s_hist[t];
}

__device__ __forceinline__ uint64_t lanemask_lt() {
    const int lane = threadIdx.x & (kWave - 1);
    return lane == 0 ? 0ull : (~0ull >> (kWave - lane));
}

// Stable scatter of one 4096-key tile.  Ranks are computed in the tile's
// original order (round, wave, lane) with wave ballots, staged sorted in LDS,
// then written out so that consecutive lanes store consecutive addresses of the
// same digit run.
__global__ __launch_bounds__(kSortThreads) void k_radix_scatter(
    const int *__restrict__ kin, const int *__restrict__ vin, int *__restrict__ kout,
    int *__restrict__ vout, int64_t n, int shift, const int *__restrict__ hist_scanned, int nblocks) {
    __shared__ int s_keys[kSortTile];
    __shared__ int s_vals[kSortTile];
    __shared__ int s_wave_cnt[kSortThreads / kWave][kRadixBins];
    __shared__ int s_running[kRadixBins];
    __shared__ int s_tile_start[kRadixBins];
    __shared__ int s_gbase[kRadixBins];
    __shared__ int s_wtot[kSortThreads / kWave];
    const int t = threadIdx.x, wave = t / kWave, lane = t & (kWave - 1);
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
    s_running[t] = 0;
    s_gbase[t] = hist_scanned[(int64_t)t * nblocks + blockIdx.x];
#pragma unroll
    for (int w = 0; w < kSortThreads / kWave; ++w) s_wave_cnt[w][t] = 0;

    int key[kSortItems], val[kSortItems], rank[kSortItems];
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t i = base + (int64_t)k * kSortThreads + t;
        key[k] = i < n ? kin[i] : 0;
        val[k] = i < n ? vin[i] : 0;
        rank[k] = 0;
    }
    __syncthreads();
    const uint64_t lt = lanemask_lt();
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const bool valid = base + (int64_t)k * kSortThreads + t < n;
        const int d = (key[k] >> shift) & (kRadixBins - 1);
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < kRadixBits; ++b) {
            const bool bit = (d >> b) & 1;
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        const int r = __popcll(peers & lt);
        if (valid && r == 0) s_wave_cnt[wave][d] = __popcll(peers);
        __syncthreads();
        if (valid) {
            int off = s_running[d];
            for (int w = 0; w < wave; ++w) off += s_wave_cnt[w][d];
            rank[k] = off + r;
        }
        __syncthreads();
        int add = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / kWave; ++w) {
            add += s_wave_cnt[w][t];
            s_wave_cnt[w][t] = 0;
        }
        s_running[t] += add;
        __syncthreads();
    }
    // exclusive scan of the tile's digit counts (one digit per thread)
    {
        const int c = s_running[t];
        int v = c;
#pragma unroll
        for (int dd = 1; dd < kWave; dd <<= 1) {
            const int o = __shfl_up(v, dd, kWave);
            if (lane >= dd) v += o;
        }
        if (lane == kWave - 1) s_wtot[wave] = v;
        __syncthreads();
        int off = 0;
        for (int w = 0; w < wave; ++w) off += s_wtot[w];
        s_tile_start[t] = off + v - c;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const bool valid = base + (int64_t)k * kSortThreads + t < n;
        if (valid) {
            const int d = (key[k] >> shift) & (kRadixBins - 1);
            const int pos = s_tile_start[d] + rank[k];
            s_keys[pos] = key[k];
            s_vals[pos] = val[k];
        }
    }
    __syncthreads();
    const int n_here = (int)min<int64_t>(kSortTile, n - base);
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int p = k * kSortThreads + t;
        if (p < n_here) {
            const int kk = s_keys[p];
            const int d = (kk >> shift) & (kRadixBins - 1);
            const int64_t dst = (int64_t)s_gbase[d] + (p - s_tile_start[d]);
            kout[dst] = kk;
            vout[dst] = s_vals[p];
        }
    }
}

// tile_bins[t] = [first, last+1) of tile t in the sorted keys; other tiles keep
// the zeros written before (bin_and_sort_gaussians.cu:40-62).
__global__ __launch_bounds__(256) void k_tile_edges(const int *__restrict__ keys, int64_t n,
                                                    int64_t n_tiles, int2 *__restrict__ bins) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int k = keys[i];
    if (k < 0 || k >= n_tiles) return;
    if (i == 0 || keys[i - 1] != k) bins[k].x = (int)i;
    if (i == n - 1 || keys[i + 1] != k) bins[k].y = (int)(i + 1);
}

struct BinLayout {
    size_t keys_a, vals_a, keys_b, hist, scan, total;
    int passes, nblocks;
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

BinLayout bin_layout(int64_t n_isect, int64_t n_tiles) {
    BinLayout L{};
    int bits = 0;
    while (bits < 31 && ((int64_t)1 << bits) < n_tiles) ++bits;
    L.passes = (bits + kRadixBits - 1) / kRadixBits;
    L.nblocks = (int)((n_isect + kSortTile - 1) / kSortTile);
    const size_t arr = align256((size_t)n_isect * sizeof(int));
    size_t off = 0;
    L.keys_a = off; off += arr;
    L.vals_a = off; off += arr;
    L.keys_b = off; off += arr;
    L.hist = off; off += align256((size_t)kRadixBins * L.nblocks * sizeof(int));
    L.scan = off; off += scan_workspace_bytes((int64_t)kRadixBins * L.nblocks);
    L.total = off; off += 256;
    return L;
}

}  // namespace
}  // namespace gsv

using namespace gsv;

extern "C" int gsv_bin_workspace_bytes(int32_t n, int64_t num_intersects, int32_t D, int32_t H,
                                       int32_t W, size_t *bytes) {
    if (!bytes || n < 0 || D <= 0 || H <= 0 || W <= 0) return GSV_ERR_INVALID_ARGUMENT;
    if (num_intersects > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const int64_t T = (int64_t)gsv_tiles_along(W) * gsv_tiles_along(H) * gsv_tiles_along(D);
    const BinLayout L = bin_layout(num_intersects > 0 ? num_intersects : 0, T);
    *bytes = L.total + 256;
    return GSV_OK;
}

extern "C" int gsv_bin_and_sort(int32_t n, int64_t num_intersects, const int32_t *tile_min,
                                const int32_t *tile_max, const int32_t *cum_tiles_hit, int32_t D,
                                int32_t H, int32_t W, void *workspace, size_t workspace_bytes,
                                int32_t *gaussian_ids_sorted, int32_t *tile_bins, void *stream) {
    if (n < 0 || D <= 0 || H <= 0 || W <= 0 || !tile_bins) return GSV_ERR_INVALID_ARGUMENT;
    if (num_intersects > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    const int64_t T = (int64_t)Tx * Ty * Tz;
    if (T > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    hipStream_t s = as_stream(stream);
    if (int st = fill_zero_u32(tile_bins, 2 * T, s)) return st;
    if (num_intersects <= 0 || n == 0) return GSV_OK;
    if (!tile_min || !tile_max || !cum_tiles_hit || !gaussian_ids_sorted || !workspace)
        return GSV_ERR_INVALID_ARGUMENT;
    const int64_t I = num_intersects;
    const BinLayout L = bin_layout(I, T);
    if (workspace_bytes < L.total + 256) return GSV_ERR_WORKSPACE_TOO_SMALL;
    char *ws = static_cast<char *>(workspace);
    int *ka = reinterpret_cast<int *>(ws + L.keys_a);
    int *va = reinterpret_cast<int *>(ws + L.vals_a);
    int *kb = reinterpret_cast<int *>(ws + L.keys_b);
    int *vb = gaussian_ids_sorted;
    int *hist = reinterpret_cast<int *>(ws + L.hist);
    // Emit into the pair of buffers that leaves the final pass in (kb, vb).
    int *kin = (L.passes % 2 == 0) ? kb : ka;
    int *vin = (L.passes % 2 == 0) ? vb : va;
    hipLaunchKernelGGL(k_emit, dim3((n + kEmitThreads - 1) / kEmitThreads), dim3(kEmitThreads), 0,
                       s, n, I, tile_min, tile_max, cum_tiles_hit, Tx, Ty, kin, vin);
    if (int st = check_launch()) return st;
    for (int p = 0; p < L.passes; ++p) {
        int *kout = (kin == ka) ? kb : ka;
        int *vout = (vin == va) ? vb : va;
        const int shift = p * kRadixBits;
        hipLaunchKernelGGL(k_radix_hist, dim3(L.nblocks), dim3(kSortThreads), 0, s, kin, I, shift,
                           hist, L.nblocks);
        if (int st = check_launch()) return st;
        if (int st = scan_i32(hist, hist, (int64_t)kRadixBins * L.nblocks, false, nullptr,
                              ws + L.scan, scan_workspace_bytes((int64_t)kRadixBins * L.nblocks), s))
            return st;
        hipLaunchKernelGGL(k_radix_scatter, dim3(L.nblocks), dim3(kSortThreads), 0, s, kin, vin,
                           kout, vout, I, shift, hist, L.nblocks);
        if (int st = check_launch()) return st;
        kin = kout;
        vin = vout;
    }
    hipLaunchKernelGGL(k_tile_edges, dim3((unsigned)((I + 255) / 256)), dim3(256), 0, s, kin, I, T,
                       reinterpret_cast<int2 *>(tile_bins));
    return check_launch();
}
