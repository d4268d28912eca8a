// binning.hip — (tile, gaussian) key duplication, a stable sort over the
// significant tile-id bits, and tile-range extraction, for gfx950.
//
// Reference: gs_voxelizer/cuda/bin_and_sort_gaussians.cu:11-62 and the binding
// bindings.cu:259-360 (which sorts all 32 key bits with cub::DeviceRadixSort).
// Keys are tile ids < T, so only bits = ceil(log2 T) bits are sorted (15 at
// 256^3, 18 at 512^3).  Because the keys are emitted gaussian-major and every
// step is stable, the result is the reference's exact order: ascending tile,
// then ascending gaussian id.  Two paths give the same bits:
//
// Bucket path (padded keys of up to 18 bits, up to ~40k pairs of capacity per
// bucket on average: 256^3 / 200k, 512^3 / 1M), four launches.  It sorts
// padded keys (tile row << xb | tx, 2^xb >= Tx), which order the pairs as the
// tile ids do, and whose low bits hold whole tile rows, so that each row of a
// Gaussian's box falls in one bucket:
//   k_bucket_hist    per chunk of 256 Gaussians, its pair count per top digit
//                    (8 bits, 9 for 17-bit keys, 10 for 18-bit ones), from the
//                    boxes' rows (no pair is emitted);
//   k_digit_scan     one block per digit: exclusive prefix of the per-chunk
//                    counts over chunks, plus the digit total;
//   k_bucket_split   stable split of the chunk's box rows by top digit, each
//                    row ranked once and expanded into one packed word per
//                    pair (gaussian << lb | the lb low key bits), so that every
//                    bucket of 2^lb keys is one contiguous run;
//   k_bucket_sort    one 1024-thread block per bucket sorts it by the low bits
//                    in LDS and writes ids, tiles and tile_bins.
// These read cum and the boxes, never the pair count: slots at or above the
// capacity are left out.  When one call also runs the prefix sum of
// num_tiles_hit (gsv_cumsum_bin_and_sort_device_count), the first two become
// extra blocks of the scan's two launches (k_sums_hist, k_apply_digits): the
// prefix sum and the binning in four launches.  Emission slots past a Gaussian's box (a cum that
// disagrees with the boxes, which the reference does not guard against either)
// carry the all-ones key and no tile on both paths; the sorts order only the
// significant key bits, so where those name a real tile (all key bits in use)
// such slots fall among or after that tile's pairs.
// LSD path (wider keys, heavier buckets), 7 launches for two passes:
//   k_emit_chunk     block b writes emission slots [4096 b, 4096 b + 4096) and
//                    that chunk's histogram of the lowest digit; it also
//                    zero-fills tile_bins;
//   k_digit_scan, k_radix_scatter (keys and ids) per pass;
//   k_radix_hist     per-chunk digit histogram for the later passes;
//   k_tile_edges     [start, end) per tile, 16 sorted keys per thread.
// Every LSD kernel reads the live pair count from device memory when one is
// given (capped by the capacity its grid was sized for), so the host need not
// know the count before launching.
//
// Data movement per pair, bucket path: the split writes 4 B, the bucket sort
// reads 4 B and writes 8 B (4 without the tiles); the boxes are read twice
// (28 B per Gaussian each time).  LSD path: emission writes 8 B; each pass
// reads 8 B and writes 8 B (later passes read 4 B more for the histogram); the
// range pass reads 4 B.
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "gsv_device.h"
#include "gsv_scan.h"

namespace gsv {
namespace {

constexpr int kChunk = 4096;  // keys per emission chunk and per scatter block
constexpr int kEmitThreads = 512;
constexpr int kEmitItems = kChunk / kEmitThreads;  // 8 consecutive slots per thread
constexpr int kWindow = 1024;                       // Gaussians cached by an emission block
constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kWaveKeys = kChunk / kSortWaves;  // 1024 contiguous keys per wave
constexpr int kRounds = kWaveKeys / kWave;      // 16
// Digit width of the LSD passes: 8 bits, or 9 when that saves a pass (keys of
// 17 or 18 bits: two 9-bit passes instead of 8 + 8 + 1..2).  Arrays shared by
// the passes are sized for the widest digit.
constexpr int kRadixBitsMax = 9;
constexpr int kRadixBinsMax = 1 << kRadixBitsMax;
constexpr int kEdgeItems = 16;
constexpr int kRemapChunks = 2048;  // XCD-contiguous scatter chunks above 8M pairs
constexpr int kInvalidKey = 0x7fffffff;  // slot beyond its Gaussian's box: sorts last, no tile
static_assert(kRadixBinsMax % kSortThreads == 0, "whole rounds of digits per thread");
static_assert(kRadixBinsMax <= kEmitThreads, "one digit per emission thread");
static_assert(kEmitItems == 8, "two int4 stores per thread");

__device__ __forceinline__ int64_t live_count(int64_t cap, const int64_t *d_n) {
    if (!d_n) return cap;
    const int64_t v = *d_n;
    return v < 0 ? 0 : (v < cap ? v : cap);
}

// Block b writes the emission slots [b*kChunk, (b+1)*kChunk) of the pairs:
// Gaussian-major, and for each Gaussian its box tiles z -> y -> x with x
// fastest (bin_and_sort_gaussians.cu:11-35).  Slot p belongs to the Gaussian g
// with cum[g-1] <= p < cum[g].  The block finds the first such Gaussian with a
// 512-way cooperative search of cum, caches cum and the tile boxes of the
// Gaussians that follow in LDS (in rounds of 512 until they cover the chunk,
// at most kWindow; beyond that it reads global memory), and gives each thread
// 8 consecutive slots: one search and one division per thread, then stepping
// through the box.  The chunk's histogram of the first pass's digit, bits
// [shift, shift + B) of the key, is written digit-major: hist[d * hstride + b].
// tile_bins (when given) is zero-filled for k_tile_edges.
template <int B>
__global__ __launch_bounds__(kEmitThreads) void k_emit_chunk(
    int n, int64_t cap, const int64_t *__restrict__ d_n, const int *__restrict__ tile_min,
    const int *__restrict__ tile_max, const int *__restrict__ cum, int Tx, int Ty, int64_t T,
    int *__restrict__ keys, int *__restrict__ vals, int *__restrict__ hist, int hstride,
    int shift, int2 *__restrict__ tile_bins) {
    __shared__ int s_cum[kWindow];
    constexpr int kBins = 1 << B;
    __shared__ int s_box[kWindow][6];  // min x, y, z; extent x, y, z
    __shared__ int s_hist[kBins];
    const int t = threadIdx.x;
    if (tile_bins != nullptr)
        for (int64_t i = (int64_t)blockIdx.x * kEmitThreads + t; i < T;
             i += (int64_t)gridDim.x * kEmitThreads)
            tile_bins[i] = make_int2(0, 0);
    if (t < kBins) s_hist[t] = 0;
    const int64_t total = live_count(cap, d_n);
    const int64_t base = (int64_t)blockIdx.x * kChunk;

    // g_lo = min{g : cum[g] > base}, or n.  Invariant: cum[g] <= base for g < lo,
    // and hi == n or cum[hi] > base.  Each round probes kEmitThreads points of
    // [lo, hi) and keeps the interval between the last "<=" and the first ">".
    int lo = 0, hi = n;
    if (base < total) {
        while (lo < hi) {
            const int64_t span = hi - lo;
            const int q = lo + (int)((span * t) / kEmitThreads);
            const int c = __syncthreads_count(cum[q] <= base);
            if (c == 0) { hi = lo; break; }
            const int qa = lo + (int)((span * (c - 1)) / kEmitThreads);
            const int qb = c < kEmitThreads ? lo + (int)((span * c) / kEmitThreads) : hi;
            lo = qa + 1;
            hi = qb > lo ? qb : lo;
        }
    }
    const int g_lo = lo;
    const int avail = base < total ? min(kWindow, n - g_lo) : 0;
    const int64_t chunk_last = min<int64_t>(base + kChunk, total) - 1;
    int wlen = 0;
    for (int r = 0; r * kEmitThreads < avail; ++r) {  // uniform: avail and LDS reads agree
        const int i = r * kEmitThreads + t;
        if (i < avail) {
            const int g = g_lo + i;
            s_cum[i] = cum[g];
            const int mnx = tile_min[3 * g], mny = tile_min[3 * g + 1], mnz = tile_min[3 * g + 2];
            s_box[i][0] = mnx; s_box[i][1] = mny; s_box[i][2] = mnz;
            s_box[i][3] = tile_max[3 * g] - mnx;
            s_box[i][4] = tile_max[3 * g + 1] - mny;
            s_box[i][5] = tile_max[3 * g + 2] - mnz;
        }
        wlen = min((r + 1) * kEmitThreads, avail);
        __syncthreads();
        if ((int64_t)s_cum[wlen - 1] > chunk_last) break;
    }
    const int prev = g_lo > 0 ? cum[g_lo - 1] : 0;
    __syncthreads();

    const int64_t p0 = base + (int64_t)t * kEmitItems;
    if (p0 < total) {
        // 32-bit slot arithmetic from here: p0 < total <= cap <= INT32_MAX, and
        // slot p0 + k is only formed for k < rem
        const int q0 = (int)p0, rem = (int)(total - p0);
        // cum and box at window index i (global memory beyond the window)
        auto cum_at = [&](int i) -> int { return i < wlen ? s_cum[i] : cum[g_lo + i]; };
        int mnx = 0, mny = 0, mnz = 0, ex = 0, ey = 0, ez = 0, dx = 0, dy = 0, dz = 0;
        auto load_box = [&](int i) {  // the box of window index i, stepping from its first tile
            if (i < wlen) {
                mnx = s_box[i][0]; mny = s_box[i][1]; mnz = s_box[i][2];
                ex = s_box[i][3]; ey = s_box[i][4]; ez = s_box[i][5];
            } else {
                const int g = g_lo + i;
                mnx = tile_min[3 * g]; mny = tile_min[3 * g + 1]; mnz = tile_min[3 * g + 2];
                ex = tile_max[3 * g] - mnx; ey = tile_max[3 * g + 1] - mny;
                ez = tile_max[3 * g + 2] - mnz;
            }
            dx = dy = dz = 0;
        };
        // l = min{i : cum_at(i) > q0}, searched in the window, then beyond it
        int l;
        if (wlen > 0 && s_cum[wlen - 1] > q0) {
            int a = 0, b = wlen - 1;
            while (a < b) {
                const int m = (a + b) >> 1;
                if (s_cum[m] > q0) b = m; else a = m + 1;
            }
            l = a;
        } else {
            int a = wlen, b = n - g_lo;  // answer in [wlen, n - g_lo]
            while (a < b) {
                const int m = (a + b) >> 1;
                if (cum[g_lo + m] > q0) b = m; else a = m + 1;
            }
            l = a;
        }
        int key[kEmitItems], val[kEmitItems];
        int g = g_lo + l;
        int start = l == 0 ? prev : cum_at(l - 1);
        int end = g < n ? cum_at(l) : start;
        if (g < n) {  // the thread's first slot may lie inside the box: one division
            load_box(l);
            const int j = q0 - start;
            if (ex > 0 && ey > 0 && ez > 0) {
                const unsigned r = (unsigned)j / (unsigned)ex;
                dx = j - (int)r * ex;
                dy = (int)(r % (unsigned)ey);
                dz = (int)(r / (unsigned)ey);
            }
        }
#pragma unroll
        for (int k = 0; k < kEmitItems; ++k) {
            if (k >= rem || g >= n) {
                key[k] = kInvalidKey;
                val[k] = 0;
                continue;
            }
            const int p = q0 + k;
            if (p >= end) {  // next non-empty Gaussian; p is its first slot (p == start)
                do {
                    ++l;
                    ++g;
                    start = end;
                    end = g < n ? cum_at(l) : start;
                } while (g < n && p >= end);
                if (g >= n) { key[k] = kInvalidKey; val[k] = 0; continue; }
                load_box(l);
            }
            val[k] = g;
            // a slot past the box (cum inconsistent with the box) gets no tile
            key[k] = (ex > 0 && ey > 0 && dz < ez)
                         ? (mnz + dz) * Ty * Tx + (mny + dy) * Tx + (mnx + dx)
                         : kInvalidKey;
            if (++dx == ex) { dx = 0; if (++dy == ey) { dy = 0; ++dz; } }
        }
        // slots [p0, p0 + 8): two 16-byte stores when whole
        if (p0 + kEmitItems <= total) {
            int4 *k4 = reinterpret_cast<int4 *>(keys + p0);
            int4 *v4 = reinterpret_cast<int4 *>(vals + p0);
            k4[0] = make_int4(key[0], key[1], key[2], key[3]);
            k4[1] = make_int4(key[4], key[5], key[6], key[7]);
            v4[0] = make_int4(val[0], val[1], val[2], val[3]);
            v4[1] = make_int4(val[4], val[5], val[6], val[7]);
        } else {
#pragma unroll
            for (int k = 0; k < kEmitItems; ++k)
                if (p0 + k < total) { keys[p0 + k] = key[k]; vals[p0 + k] = val[k]; }
        }
#pragma unroll
        for (int k = 0; k < kEmitItems; ++k)
            if (p0 + k < total) atomicAdd(&s_hist[(key[k] >> shift) & (kBins - 1)], 1);
    }
    __syncthreads();
    if (t < kBins) hist[(int64_t)t * hstride + blockIdx.x] = s_hist[t];
}

// Per-chunk digit histogram of a later pass, digit-major; chunks past the live
// count write zeros.
template <int B>
__global__ __launch_bounds__(kSortThreads) void k_radix_hist(const int *__restrict__ keys,
                                                             int64_t cap,
                                                             const int64_t *__restrict__ d_n,
                                                             int shift, int *__restrict__ hist,
                                                             int hstride) {
    constexpr int kBins = 1 << B;
    __shared__ int s_hist[kBins];
    const int t = threadIdx.x;
#pragma unroll
    for (int d = t; d < kBins; d += kSortThreads) s_hist[d] = 0;
    __syncthreads();
    const int64_t n = live_count(cap, d_n);
    const int64_t base = (int64_t)blockIdx.x * kChunk;
#pragma unroll
    for (int q = 0; q < kChunk / kSortThreads / 4; ++q) {
        const int64_t i = base + 4 * ((int64_t)q * kSortThreads + t);
        if (i + 4 <= n) {
            const int4 k4 = *reinterpret_cast<const int4 *>(keys + i);
            atomicAdd(&s_hist[(k4.x >> shift) & (kBins - 1)], 1);
            atomicAdd(&s_hist[(k4.y >> shift) & (kBins - 1)], 1);
            atomicAdd(&s_hist[(k4.z >> shift) & (kBins - 1)], 1);
            atomicAdd(&s_hist[(k4.w >> shift) & (kBins - 1)], 1);
        } else {
            for (int64_t j = i; j < n && j < i + 4; ++j)
                atomicAdd(&s_hist[(keys[j] >> shift) & (kBins - 1)], 1);
        }
    }
    __syncthreads();
#pragma unroll
    for (int d = t; d < kBins; d += kSortThreads)
        hist[(int64_t)d * hstride + blockIdx.x] = s_hist[d];
}

// Exclusive scan of one value per thread across an NT-thread block; *total
// gets the block's sum.  s_wtot holds NT / 64 values (int, or long long where
// the sum may pass 2^31).
template <int NT, typename V = int>
__device__ __forceinline__ V block_scan_total(V v, V *s_wtot, V *total) {
    const int t = threadIdx.x, wave = t / kWave, lane = t & (kWave - 1);
    V inc = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const V o = __shfl_up(inc, d, kWave);
        if (lane >= d) inc += o;
    }
    if (lane == kWave - 1) s_wtot[wave] = inc;
    __syncthreads();
    V off = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < NT / kWave; ++w) {
        const V x = s_wtot[w];
        off += w < wave ? x : 0;
        sum += x;
    }
    *total = sum;
    return off + inc - v;
}

// Block d turns hist[d][0..nblocks) into its exclusive prefix over chunks and
// writes the digit total.  The row (16-byte aligned: hstride is a multiple of
// 4) is scanned in tiles of 8192: thread t loads 8 consecutive counts with two
// 16-byte loads, one block scan gives the offsets, and the 8 prefixes go back
// with two 16-byte stores, so every access is coalesced.
constexpr int kDigitScanThreads = 1024;
constexpr int kDigitScanItems = 8;

// The scan of one digit's row by a workgroup of NT threads (s_wtot: NT / 64
// ints), in tiles of NT * 8; *total_slot gets the row's total.
template <int NT>
__device__ __forceinline__ void digit_scan_row(int *__restrict__ row, int nblocks,
                                               int *__restrict__ total_slot, int *s_wtot) {
    constexpr int kTileItems = NT * kDigitScanItems;
    int carry = 0;
    for (int base = 0; base < nblocks; base += kTileItems) {
        const int i0 = base + (int)threadIdx.x * kDigitScanItems;
        int v[kDigitScanItems];
        const bool whole = i0 + kDigitScanItems <= nblocks;
        if (whole) {
            const int4 a = *reinterpret_cast<const int4 *>(row + i0);
            const int4 b = *reinterpret_cast<const int4 *>(row + i0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int k = 0; k < kDigitScanItems; ++k) v[k] = i0 + k < nblocks ? row[i0 + k] : 0;
        }
        int s = 0;
#pragma unroll
        for (int k = 0; k < kDigitScanItems; ++k) s += v[k];
        int total;
        int run = carry + block_scan_total<NT>(s, s_wtot, &total);
        int o[kDigitScanItems];
#pragma unroll
        for (int k = 0; k < kDigitScanItems; ++k) {
            o[k] = run;
            run += v[k];
        }
        if (whole) {
            *reinterpret_cast<int4 *>(row + i0) = make_int4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<int4 *>(row + i0 + 4) = make_int4(o[4], o[5], o[6], o[7]);
        } else {
#pragma unroll
            for (int k = 0; k < kDigitScanItems; ++k)
                if (i0 + k < nblocks) row[i0 + k] = o[k];
        }
        carry += total;
        __syncthreads();  // s_wtot is rewritten by the next tile's scan
    }
    if (threadIdx.x == 0) *total_slot = carry;
}

__global__ __launch_bounds__(kDigitScanThreads) void k_digit_scan(int *__restrict__ hist,
                                                                  int nblocks, int hstride,
                                                                  int *__restrict__ totals) {
    __shared__ int s_wtot[kDigitScanThreads / kWave];
    digit_scan_row<kDigitScanThreads>(hist + (int64_t)blockIdx.x * hstride, nblocks,
                                      totals + blockIdx.x, s_wtot);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
    const int lane = threadIdx.x & (kWave - 1);
    return lane == 0 ? 0ull : (~0ull >> (kWave - lane));
}

// Exclusive scan of one int per thread across the 256-thread block.
__device__ __forceinline__ int block_excl_scan(int v, int *s_wtot) {
    int total;
    return block_scan_total<kSortThreads>(v, s_wtot, &total);
}

// Stable scatter of one 4096-key chunk.  Wave w owns keys [w*1024, (w+1)*1024)
// of the chunk and ranks them round by round (64 keys a round) against its own
// running digit counts in LDS; after one barrier the per-wave counts become
// offsets, keys are staged digit-sorted in LDS and written out so that
// consecutive lanes store consecutive addresses of the same digit run.
// With `remap`, chunks are dealt to the XCDs in contiguous ranges (xcd_remap):
// the runs of one digit from consecutive chunks are adjacent in the output, so
// their partial cache lines meet in the same L2 and reach HBM as whole lines.
// That pays once the arrays outgrow the last-level cache (~15 % of the sort at
// 30M pairs) and costs ~1 us per pass below it, where it is left off.
// With 9-bit digits each thread handles digits t and t + 256 in the per-digit
// steps; the block scans over digits then run in two rounds.
template <int B>
__global__ __launch_bounds__(kSortThreads) void k_radix_scatter(
    const int *__restrict__ kin, const int *__restrict__ vin, int *__restrict__ kout,
    int *__restrict__ vout, int64_t cap, const int64_t *__restrict__ d_n, int shift,
    const int *__restrict__ hist_scanned, const int *__restrict__ totals, int nblocks,
    int hstride, int remap) {
    constexpr int kBins = 1 << B;
    constexpr int kPer = kBins / kSortThreads;  // digits per thread in the per-digit steps
    __shared__ int s_keys[kChunk];
    __shared__ int s_vals[kChunk];
    __shared__ int s_wcnt[kSortWaves][kBins];
    __shared__ int s_start[kBins];
    __shared__ int s_gbase[kBins];
    __shared__ int s_wtot[kSortWaves];
    const int t = threadIdx.x, wave = t / kWave, lane = t & (kWave - 1);
    const int64_t n = live_count(cap, d_n);
    const int64_t chunk = remap ? xcd_remap(blockIdx.x, xcd_per(nblocks)) : blockIdx.x;
    if (chunk >= nblocks) return;
    const int64_t base = chunk * kChunk;
    if (base >= n) return;
#pragma unroll
    for (int j = 0; j < kPer; ++j)
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) s_wcnt[w][j * kSortThreads + t] = 0;
    {   // global start of this chunk's run of each digit
        int carry = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int d = j * kSortThreads + t;
            int tot;
            const int dbase = carry + block_scan_total<kSortThreads>(totals[d], s_wtot, &tot);
            s_gbase[d] = dbase + hist_scanned[(int64_t)d * hstride + chunk];
            carry += tot;
            __syncthreads();  // s_wtot is rewritten by the next round
        }
    }

    const int64_t wbase = base + (int64_t)wave * kWaveKeys;
    int key[kRounds], val[kRounds], rank[kRounds];
#pragma unroll
    for (int k = 0; k < kRounds; ++k) {
        const int64_t i = wbase + k * kWave + lane;
        key[k] = i < n ? kin[i] : 0;
        val[k] = i < n ? vin[i] : 0;
    }
    const uint64_t lt = lanemask_lt();
#pragma unroll
    for (int k = 0; k < kRounds; ++k) {
        const bool valid = wbase + k * kWave + lane < n;
        const int d = (key[k] >> shift) & (kBins - 1);
        // peers = the valid lanes whose digit equals d: per bit b, t = -1 where
        // bit b of d is set, and a lane keeps the lanes whose ballot bit agrees
        // (sign-extended bit, xor, and-not: about 6 VALU per bit, against 9
        // for a per-lane select between m and ~m)
        const uint64_t vm = __ballot(valid);
        uint32_t plo = (uint32_t)vm, phi = (uint32_t)(vm >> 32);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const uint32_t t = (uint32_t)__builtin_amdgcn_sbfe(d, b, 1);
            const uint64_t m = __ballot(t != 0u);
            plo &= ~((uint32_t)m ^ t);
            phi &= ~((uint32_t)(m >> 32) ^ t);
        }
        const uint64_t peers = ((uint64_t)phi << 32) | plo;
        const int r = __popcll(peers & lt);
        // one wave reads then updates its own counters: LDS keeps the order
        const int off = s_wcnt[wave][d];
        rank[k] = off + r;
        if (valid && r == 0) s_wcnt[wave][d] = off + __popcll(peers);
    }
    __syncthreads();
    {   // per-digit wave offsets, then the chunk's digit starts
        int sum[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int d = j * kSortThreads + t;
            sum[j] = 0;
#pragma unroll
            for (int w = 0; w < kSortWaves; ++w) {
                const int c = s_wcnt[w][d];
                s_wcnt[w][d] = sum[j];
                sum[j] += c;
            }
        }
        int carry = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            __syncthreads();  // s_wtot is rewritten by this round's scan
            int tot;
            s_start[j * kSortThreads + t] =
                carry + block_scan_total<kSortThreads>(sum[j], s_wtot, &tot);
            carry += tot;
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kRounds; ++k) {
        if (wbase + k * kWave + lane < n) {
            const int d = (key[k] >> shift) & (kBins - 1);
            const int pos = s_start[d] + s_wcnt[wave][d] + rank[k];
            s_keys[pos] = key[k];
            s_vals[pos] = val[k];
        }
    }
    __syncthreads();
    const int n_here = (int)min<int64_t>(kChunk, n - base);
#pragma unroll
    for (int k = 0; k < kChunk / kSortThreads; ++k) {
        const int p = k * kSortThreads + t;
        if (p < n_here) {
            const int kk = s_keys[p];
            const int d = (kk >> shift) & (kBins - 1);
            const int64_t dst = (int64_t)s_gbase[d] + (p - s_start[d]);
            kout[dst] = kk;
            vout[dst] = s_vals[p];
        }
    }
}

// tile_bins[t] = [first, last+1) of tile t in the sorted keys; tiles without
// pairs keep the zeros k_emit_chunk wrote (bin_and_sort_gaussians.cu:40-62).
__global__ __launch_bounds__(256) void k_tile_edges(const int *__restrict__ keys, int64_t cap,
                                                    const int64_t *__restrict__ d_n,
                                                    int64_t n_tiles, int2 *__restrict__ bins) {
    const int64_t n = live_count(cap, d_n);
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kEdgeItems;
    if (i0 >= n) return;
    int k[kEdgeItems + 1];
    if (i0 + kEdgeItems <= n) {
        const int4 *k4 = reinterpret_cast<const int4 *>(keys + i0);
#pragma unroll
        for (int q = 0; q < kEdgeItems / 4; ++q) {
            const int4 v = k4[q];
            k[4 * q] = v.x; k[4 * q + 1] = v.y; k[4 * q + 2] = v.z; k[4 * q + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < kEdgeItems; ++q) k[q] = i0 + q < n ? keys[i0 + q] : kInvalidKey;
    }
    k[kEdgeItems] = i0 + kEdgeItems < n ? keys[i0 + kEdgeItems] : kInvalidKey;
    int before = i0 > 0 ? keys[i0 - 1] : kInvalidKey;
#pragma unroll
    for (int q = 0; q < kEdgeItems; ++q) {
        const int64_t i = i0 + q;
        const int kk = k[q];
        if (i < n && kk >= 0 && kk < n_tiles) {
            if (before != kk) bins[kk].x = (int)i;
            if (i == n - 1 || k[q + 1] != kk) bins[kk].y = (int)(i + 1);
        }
        before = kk;
    }
}

// ------------------------------------------------ bucket path: box rows --
//
// The bucket path sorts padded keys, key = row << xb | tx with row = tz * Ty +
// ty and 2^xb the tile count along x rounded up to a power of two.  Tile id ->
// padded key is increasing, so both give the same order.  The low lb >= xb
// bits of a key hold whole rows, so every row of a Gaussian's box lies in one
// bucket (top digit = key >> lb), and the emission order of a Gaussian's pairs
// (its box z -> y -> x) is a sequence of rows of ex consecutive tiles.  The
// split into buckets therefore works on rows: a row is one entry with one
// digit and a weight of ex pairs, never a pair at a time.
struct BucketGeom {
    int Tx, Ty;  // tiles along x and y
    int rows;    // Ty * Tz
    int xb;      // bits of the padded x coordinate
    int lb;      // low key bits sorted inside a bucket (xb <= lb <= 9)
    int nbits;   // top digit bits: 2^nbits buckets
};

// One Gaussian's emitted slots [cum[g-1], cum[g]) below the capacity, as box
// rows: the first nvalid slots are the box's tiles z -> y -> x (nvalid =
// min(slots, box volume)); the remaining ninvalid slots (only when cum
// disagrees with the box) carry no tile and sort last.
struct GaussRows {
    int mnx, mny, mnz, ex, ey;
    int nvalid, ninvalid, nrows;
};

__device__ __forceinline__ GaussRows gauss_rows(int g, int n, int64_t cap,
                                                const int *__restrict__ tile_min,
                                                const int *__restrict__ tile_max,
                                                const int *__restrict__ cum) {
    GaussRows r{};
    if (g >= n) return r;
    // ns in [0, cap] even where an int32 cum has wrapped past 2^31 (s0 < 0)
    const int64_t s0 = g > 0 ? cum[g - 1] : 0;
    const int64_t s1 = min<int64_t>(cum[g], cap);
    const int64_t ns = s1 > s0 ? min(s1 - s0, cap) : 0;
    r.mnx = tile_min[3 * g]; r.mny = tile_min[3 * g + 1]; r.mnz = tile_min[3 * g + 2];
    r.ex = tile_max[3 * g] - r.mnx;
    r.ey = tile_max[3 * g + 1] - r.mny;
    const int ez = tile_max[3 * g + 2] - r.mnz;
    const int64_t vol = (r.ex > 0 && r.ey > 0 && ez > 0) ? (int64_t)r.ex * r.ey * ez : 0;
    const int64_t nv = min(ns, vol);
    r.nvalid = (int)nv;
    r.ninvalid = (int)(ns - nv);
    r.nrows = nv > 0 ? (int)((nv + r.ex - 1) / r.ex) : 0;
    return r;
}

// Padded key of the first tile of box row (dz, dy); unsigned arithmetic, so a
// box outside the grid gives a wrong but in-range digit, never a fault.
__device__ __forceinline__ unsigned row_key(const BucketGeom &G, int mnx, int mny, int mnz, int dz,
                                            int dy) {
    const unsigned row = (unsigned)(mnz + dz) * (unsigned)G.Ty + (unsigned)(mny + dy);
    return (row << G.xb) | (unsigned)mnx;
}

constexpr int kSplitThreads = 256;  // Gaussians per chunk of the bucket split
constexpr int kSplitWaves = kSplitThreads / kWave;
constexpr int kPiece = 512;  // entries a split wave lists at a time

// Adds the lane's Gaussian's pairs to h[top digit]: one atomic per run of
// rows with one digit (a run of 2^(lb - xb) rows at most), plus the slots
// past the box to the last digit.
__device__ __forceinline__ void add_row_counts(const BucketGeom &G, const GaussRows &r, int nb,
                                               int *h) {
    int cur = 0, acc = 0, dz = 0, dy = 0;
    for (int q = 0; q < r.nrows; ++q) {
        const int d = (int)((row_key(G, r.mnx, r.mny, r.mnz, dz, dy) >> G.lb) & (unsigned)(nb - 1));
        if (d != cur && acc) {
            atomicAdd(&h[cur], acc);
            acc = 0;
        }
        cur = d;
        acc += min(r.ex, r.nvalid - q * r.ex);
        if (++dy == r.ey) { dy = 0; ++dz; }
    }
    if (acc) atomicAdd(&h[cur], acc);
    if (r.ninvalid) atomicAdd(&h[nb - 1], r.ninvalid);
}

// Pass 1: chunk c = the kSplitThreads Gaussians from kSplitThreads * c, one
// lane each; the chunk's pair count per top digit, hist[d * hstride + c]
// (digit-major, as k_digit_scan takes it).
template <int Bt>
__global__ __launch_bounds__(kSplitThreads) void k_bucket_hist(
    int n, int64_t cap, const int *__restrict__ tile_min, const int *__restrict__ tile_max,
    const int *__restrict__ cum, BucketGeom G, int *__restrict__ hist, int hstride) {
    __shared__ int s_h[1 << Bt];
    const int t = threadIdx.x, nb = 1 << G.nbits;
    for (int d = t; d < nb; d += kSplitThreads) s_h[d] = 0;
    __syncthreads();
    const GaussRows r = gauss_rows(blockIdx.x * kSplitThreads + t, n, cap, tile_min, tile_max, cum);
    add_row_counts(G, r, nb, s_h);
    __syncthreads();
    for (int d = t; d < nb; d += kSplitThreads) hist[(int64_t)d * hstride + blockIdx.x] = s_h[d];
}

// ------------------------------------ prefix sum and bucket counts fused --
//
// When one call runs the prefix sum of num_tiles_hit and the binning
// (gsv_cumsum_bin_and_sort_device_count), the bucket path's two small passes
// ride on the scan's two launches: the chunks' bucket counts beside the scan's
// block sums (they need the boxes and the tile counts, not the prefix sum),
// the prefix over chunks beside the scan's apply pass.  Four launches for the
// prefix sum and the binning instead of six; the same words, ids and bins.

// A Gaussian's rows from its tile count instead of cum: equal to gauss_rows
// (ns = cum[g] - cum[g-1] = num_tiles_hit[g]) whenever the pairs fit the
// capacity.  Past it the binning's output is incomplete whichever counts it
// uses, and the caller runs it again; every store stays guarded by cap.
__device__ __forceinline__ GaussRows gauss_rows_nth(int g, int n, const int *__restrict__ nth,
                                                    const int *__restrict__ tile_min,
                                                    const int *__restrict__ tile_max) {
    GaussRows r{};
    if (g >= n) return r;
    const int64_t ns = nth[g] > 0 ? nth[g] : 0;
    r.mnx = tile_min[3 * g]; r.mny = tile_min[3 * g + 1]; r.mnz = tile_min[3 * g + 2];
    r.ex = tile_max[3 * g] - r.mnx;
    r.ey = tile_max[3 * g + 1] - r.mny;
    const int ez = tile_max[3 * g + 2] - r.mnz;
    const int64_t vol = (r.ex > 0 && r.ey > 0 && ez > 0) ? (int64_t)r.ex * r.ey * ez : 0;
    const int64_t nv = min(ns, vol);
    r.nvalid = (int)nv;
    r.ninvalid = (int)(ns - nv);
    r.nrows = nv > 0 ? (int)((nv + r.ex - 1) / r.ex) : 0;
    return r;
}

static_assert(kSplitThreads == scan_detail::kThreads, "one block size for both halves");

// Blocks [0, nb_scan): the scan's block sums of num_tiles_hit; blocks
// nb_scan + c: chunk c's bucket counts, as k_bucket_hist.
template <int Bt>
__global__ __launch_bounds__(kSplitThreads) void k_sums_hist(
    const int32_t *__restrict__ nth, int n, int nb_scan, int32_t *__restrict__ part,
    const int *__restrict__ tile_min, const int *__restrict__ tile_max, BucketGeom G,
    int *__restrict__ hist, int hstride) {
    __shared__ int s_h[1 << Bt];
    __shared__ int lds_waves[kSplitThreads / kWave];
    if ((int)blockIdx.x < nb_scan) {  // uniform per block
        scan_detail::block_sums_body(LoadI32{nth}, (int64_t)n, part, (int)blockIdx.x, lds_waves);
        return;
    }
    const int chunk = (int)blockIdx.x - nb_scan;
    const int t = threadIdx.x, nb = 1 << G.nbits;
    for (int d = t; d < nb; d += kSplitThreads) s_h[d] = 0;
    __syncthreads();
    const GaussRows r = gauss_rows_nth(chunk * kSplitThreads + t, n, nth, tile_min, tile_max);
    add_row_counts(G, r, nb, s_h);
    __syncthreads();
    for (int d = t; d < nb; d += kSplitThreads) hist[(int64_t)d * hstride + chunk] = s_h[d];
}

// Blocks [0, nb_scan): the scan's apply pass (cum = inclusive prefix sum, the
// total to *total_out and *total_host); blocks nb_scan + d: digit d's prefix
// over the chunks and its total, as k_digit_scan.
__global__ __launch_bounds__(kSplitThreads) void k_apply_digits(
    const int32_t *__restrict__ nth, int32_t *__restrict__ cum, int n, int nb_scan,
    const int32_t *__restrict__ part, int64_t *__restrict__ total_out, int64_t *total_host,
    int *__restrict__ hist, int nchunks, int hstride, int *__restrict__ totals) {
    __shared__ int lds_waves[kSplitThreads / kWave];
    __shared__ long long lds_pre[kSplitThreads / kWave];
    if ((int)blockIdx.x < nb_scan) {  // uniform per block
        scan_detail::apply_body(LoadI32{nth}, StoreI32{cum, 1}, (int64_t)n, part, 1, total_out,
                                total_host, (int)blockIdx.x, nb_scan, lds_waves, lds_pre);
        return;
    }
    const int d = (int)blockIdx.x - nb_scan;
    digit_scan_row<kSplitThreads>(hist + (int64_t)d * hstride, nchunks, totals + d, lds_waves);
}

// Pass 2: the stable split of chunk c.  Each wave walks its 64 Gaussians'
// rows once, counting their pairs per digit again and listing the rows in
// emission order in LDS (lane-major, kPiece at a time; later pieces are listed
// when reached).  One counter per (wave, digit) starts at the digit's start,
// plus the chunk's prefix (k_digit_scan turned hist into the prefix over
// chunks and wrote the digit totals), plus the earlier waves' counts.  The
// wave then walks its list 64 rows a round: each row
// takes its digit's counter plus the pairs of the lower lanes of the round
// with the same digit (weights summed from bit-sliced ballots), the lowest
// such lane advances the counter by the round's total, and each lane writes
// its row's words, (gaussian << lb) | the key's low lb bits.  Slots past a box
// get the all-ones key.
template <int Bt>
__global__ __launch_bounds__(kSplitThreads) void k_bucket_split(
    int n, int64_t cap, const int *__restrict__ tile_min, const int *__restrict__ tile_max,
    const int *__restrict__ cum, BucketGeom G, const int *__restrict__ hist, int hstride,
    const int *__restrict__ totals, unsigned *__restrict__ words) {
    __shared__ int s_cnt[kSplitWaves][1 << Bt];
    __shared__ int2 s_list[kSplitWaves][kPiece];
    __shared__ int s_info[kSplitWaves][7][kWave];
    __shared__ int s_wtot[kSplitWaves];
    const int t = threadIdx.x, wave = t / kWave, lane = t & (kWave - 1);
    const int chunk = blockIdx.x, nb = 1 << G.nbits;
    const unsigned lmask = (1u << G.lb) - 1u;
    // the digit totals and this chunk's prefix, loaded ahead of the counting
    constexpr int kPer = (1 << Bt) / kSplitThreads;
    int tv[kPer], hv[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int d = j * kSplitThreads + t;
        tv[j] = d < nb ? totals[d] : 0;
        hv[j] = d < nb ? hist[(int64_t)d * hstride + chunk] : 0;
    }
    for (int d = t; d < nb; d += kSplitThreads)
#pragma unroll
        for (int w = 0; w < kSplitWaves; ++w) s_cnt[w][d] = 0;
    const int g0 = chunk * kSplitThreads + wave * kWave;
    const GaussRows r = gauss_rows(g0 + lane, n, cap, tile_min, tile_max, cum);
    int *cnt = s_cnt[wave];
    int *info = &s_info[wave][0][0];
    info[0 * kWave + lane] = r.mnx;
    info[1 * kWave + lane] = r.mny;
    info[2 * kWave + lane] = r.mnz;
    info[3 * kWave + lane] = r.ex;
    info[4 * kWave + lane] = r.ey;
    info[5 * kWave + lane] = r.nvalid;
    info[6 * kWave + lane] = r.ninvalid;
    const int nent = r.nrows + (r.ninvalid > 0 ? 1 : 0);
    int ent_inc = nent;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(ent_inc, o, kWave);
        if (lane >= o) ent_inc += v;
    }
    const int base = ent_inc - nent;
    const int E = __shfl(ent_inc, kWave - 1, kWave);
    __syncthreads();  // counters zeroed
    {   // one walk over the lane's rows: the wave's count per digit (one atomic
        // per run of rows with one digit) and the first piece of the list,
        // (lane | dy << 6, dz) per row and (lane, -1) for the slots past the box
        int cur = 0, acc = 0, dz = 0, dy = 0;
        for (int q = 0; q < r.nrows; ++q) {
            const int d =
                (int)((row_key(G, r.mnx, r.mny, r.mnz, dz, dy) >> G.lb) & (unsigned)(nb - 1));
            if (d != cur && acc) {
                atomicAdd(&cnt[cur], acc);
                acc = 0;
            }
            cur = d;
            acc += min(r.ex, r.nvalid - q * r.ex);
            if (base + q < kPiece) s_list[wave][base + q] = make_int2(lane | (dy << 6), dz);
            if (++dy == r.ey) { dy = 0; ++dz; }
        }
        if (acc) atomicAdd(&cnt[cur], acc);
        if (r.ninvalid) {
            atomicAdd(&cnt[nb - 1], r.ninvalid);
            if (base + r.nrows < kPiece) s_list[wave][base + r.nrows] = make_int2(lane, -1);
        }
    }
    __syncthreads();
    {   // counter (w, d) = start of d + chunk prefix of d + counts of waves < w
        int carry = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int d = j * kSplitThreads + t;
            int tot;
            const int dstart = carry + block_scan_total<kSplitThreads>(tv[j], s_wtot, &tot);
            carry += tot;
            if (d < nb) {
                unsigned run = (unsigned)dstart + (unsigned)hv[j];
#pragma unroll
                for (int w = 0; w < kSplitWaves; ++w) {
                    const unsigned c = (unsigned)s_cnt[w][d];
                    s_cnt[w][d] = (int)run;
                    run += c;
                }
            }
            __syncthreads();  // s_wtot is rewritten by the next round; counters final
        }
    }
    const uint64_t lt = lanemask_lt();
    for (int p0 = 0; p0 < E; p0 += kPiece) {
        if (p0 > 0) {  // this lane's entries in [p0, p0 + kPiece), as above
            const int a = max(base, p0), b = min(base + nent, p0 + kPiece);
            if (a < b) {
                int q = a - base;
                int dz = q < r.nrows ? q / r.ey : 0;
                int dy = q < r.nrows ? q - dz * r.ey : 0;
                for (int e = a; e < b; ++e, ++q) {
                    if (q < r.nrows) {
                        s_list[wave][e - p0] = make_int2(lane | (dy << 6), dz);
                        if (++dy == r.ey) { dy = 0; ++dz; }
                    } else {
                        s_list[wave][e - p0] = make_int2(lane, -1);
                    }
                }
            }
        }
        const int ne = min(kPiece, E - p0);
        for (int r0 = 0; r0 < ne; r0 += kWave) {
            const bool valid = r0 + lane < ne;
            int d = nb - 1, len = 0, src = 0;
            unsigned low = lmask, step = 0;
            if (valid) {
                const int2 en = s_list[wave][r0 + lane];
                src = en.x & (kWave - 1);
                if (en.y >= 0) {
                    const int dy = en.x >> 6, dz = en.y;
                    const int ex = info[3 * kWave + src];
                    const int q = dz * info[4 * kWave + src] + dy;
                    len = min(ex, info[5 * kWave + src] - q * ex);
                    const unsigned key = row_key(G, info[src], info[kWave + src],
                                                 info[2 * kWave + src], dz, dy);
                    d = (int)((key >> G.lb) & (unsigned)(nb - 1));
                    low = key & lmask;
                    step = 1;
                } else {
                    len = info[6 * kWave + src];
                }
            }
            // lanes of the round with the same digit
            const uint64_t vm = __ballot(valid);
            uint32_t plo = (uint32_t)vm, phi = (uint32_t)(vm >> 32);
            for (int bit = 0; bit < G.nbits; ++bit) {
                const uint32_t x = (uint32_t)__builtin_amdgcn_sbfe(d, bit, 1);
                const uint64_t m = __ballot(x != 0u);
                plo &= ~((uint32_t)m ^ x);
                phi &= ~((uint32_t)(m >> 32) ^ x);
            }
            const uint64_t peers = ((uint64_t)phi << 32) | plo;
            // their pairs below this lane (pre) and in all (tot), from as many
            // weight bits as the round's longest row needs (3 for box rows of up
            // to 7 tiles)
            unsigned pre = 0, tot = 0;  // sums below 2^31: the round's pairs are at most 64 * 2^30
            if (!__ballot(len > 7)) {
#pragma unroll
                for (int bit = 0; bit < 3; ++bit) {
                    const uint64_t m = __ballot((len >> bit) & 1) & peers;
                    pre += (unsigned)__popcll(m & lt) << bit;
                    tot += (unsigned)__popcll(m) << bit;
                }
            } else {
                for (int bit = 0; bit < 31; ++bit) {
                    const uint64_t m = __ballot((len >> bit) & 1) & peers;
                    pre += (unsigned)__popcll(m & lt) << bit;
                    tot += (unsigned)__popcll(m) << bit;
                }
            }
            const unsigned off = (unsigned)cnt[d];  // the wave's own counter: LDS keeps read-then-write order
            if (valid && __popcll(peers & lt) == 0) cnt[d] = (int)(off + tot);
            const int64_t pos = (int64_t)(int)off + (int64_t)pre;
            const unsigned gw = (unsigned)(g0 + src) << G.lb;
            if (pos >= 0 && pos + len <= cap) {  // always, unless cum disagrees with the counts
                unsigned *dst = words + pos;
                for (int k = 0; k < len; ++k) dst[k] = gw | ((low + step * (unsigned)k) & lmask);
            } else {
                for (int k = 0; k < len; ++k) {
                    const int64_t i = pos + k;
                    if (i >= 0 && i < cap) words[i] = gw | ((low + step * (unsigned)k) & lmask);
                }
            }
        }
    }
}

// Second stage of the bucket path: every bucket of 2^lb consecutive padded
// keys is one contiguous run of words (gaussian << lb | the key's low lb bits)
// in emission order; block b sorts bucket b by its low bits in LDS and writes
// the ids, the tiles (optional) and tile_bins of its tiles.
//   1. wave w counts the words of its contiguous segment per key in its own
//      row of LDS counters;
//   2. one thread per key turns the rows into per-(wave, key) offsets and the
//      tile's [start, end) (tiles without pairs get [0, 0), as the reference's
//      zero-initialised tile_bins has them; padding keys name no tile);
//   3. each wave walks its segment in order, 64 words a round: ballot-ranked
//      among the round's lanes with the same key, plus the wave's running
//      counter, which gives the stable position directly.
// A wave loads up to kBatch rounds at once (all in flight), and keeps them in
// registers from step 1 to step 3 when its segment is one batch (buckets of
// up to 18,432 pairs).  Sorted words go to LDS when the bucket fits (then
// copied out coalesced: unstaged, scattered 4-byte stores cost 22 us more at
// 256^3 / 200k), else straight to global memory (an outsized bucket of a
// clustered scene: slower, same result).  Words with the all-ones key (slots
// past a box) sort last in the last bucket.
constexpr int kBucketThreads = 1024;
constexpr int kBucketWaves = kBucketThreads / kWave;
constexpr int kBatch = 18;  // rounds of 64 words per wave and batch
static_assert((1 << kRadixBitsMax) <= kBucketThreads, "one key per thread in the offset step");

// LB: the widest low digit served (8, or 9 for 18-bit keys).  The staging
// area takes what the 160 KiB of LDS leave beside the counters: 140 KiB
// (LB = 8) or 120 KiB (LB = 9), one workgroup per CU.
template <int LB>
constexpr int kStageWords = (LB <= 8 ? 140 : 120) * 1024 / 4;

// The tile of padded key k, or kInvalidKey for a padding key.
__device__ __forceinline__ int padded_tile(const BucketGeom &G, unsigned k) {
    const unsigned row = k >> G.xb, tx = k & ((1u << G.xb) - 1u);
    return (tx < (unsigned)G.Tx && row < (unsigned)G.rows) ? (int)(row * (unsigned)G.Tx + tx)
                                                          : kInvalidKey;
}

template <int LB>
__global__ __launch_bounds__(kBucketThreads) void k_bucket_sort(
    const unsigned *__restrict__ pin, int *__restrict__ kout, int *__restrict__ vout,
    const int *__restrict__ totals, BucketGeom G, int64_t cap, int2 *__restrict__ tile_bins) {
    __shared__ int s_cnt[kBucketWaves << LB];
    __shared__ int s_wtot[kBucketWaves];
    __shared__ long long s_wtot64[kBucketWaves];
    __shared__ unsigned s_stage[kStageWords<LB>];
    const int t = threadIdx.x, wave = t / kWave, lane = t & (kWave - 1);
    const int b = blockIdx.x, lb = G.lb, nb = 1 << lb;
    const unsigned lmask = (unsigned)nb - 1u;
    // The bucket's first word: the sum of the lower buckets' totals, in 64 bits
    // and each total clamped to [0, cap].  The totals are int32 sums of the
    // pair counts; past 2^31 pairs (a call far over its capacity) they wrap,
    // and the clamps keep every access of this block inside [0, cap) whatever
    // they hold.
    auto clamp_total = [cap](int x) -> long long { return x < 0 ? 0 : min<long long>(x, cap); };
    int64_t start;
    {
        long long tot;
        block_scan_total<kBucketThreads, long long>(t < b ? clamp_total(totals[t]) : 0,
                                                    s_wtot64, &tot);
        start = min<long long>(tot, cap);
    }
    // the words below the capacity (all of them unless the counts disagree with it)
    const int size = (int)min<int64_t>(clamp_total(totals[b]), cap - start);
    for (int i = t; i < kBucketWaves * nb; i += kBucketThreads) s_cnt[i] = 0;
    // segments of whole 64-word rounds, in bucket order; batches of kBatch rounds
    const int seg = (size + kBucketWaves * kWave - 1) / (kBucketWaves * kWave) * kWave;
    const int s0 = min(wave * seg, size), s1 = min(s0 + seg, size);
    const int nbatch = (seg + kBatch * kWave - 1) / (kBatch * kWave);  // same for every wave
    const unsigned *pb = pin + start;
    int *cnt = s_cnt + wave * nb;
    unsigned w[kBatch];
    auto load = [&](int j) {
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            const int i = s0 + (j * kBatch + q) * kWave + lane;
            w[q] = i < s1 ? pb[i] : 0u;
        }
    };
    __syncthreads();  // counters zeroed; s_wtot free again
    for (int j = 0; j < nbatch; ++j) {
        load(j);
#pragma unroll
        for (int q = 0; q < kBatch; ++q)
            if (s0 + (j * kBatch + q) * kWave + lane < s1) atomicAdd(&cnt[w[q] & lmask], 1);
    }
    __syncthreads();
    const unsigned key0 = (unsigned)b << lb;
    {   // counters -> positions: one exclusive scan over (key, wave) order, the
        // 16 * 2^lb counters spread evenly over the block's threads
        static_assert(kBucketWaves == 16, "(key, wave) index = key * 16 + wave");
        const int ne = kBucketWaves * nb;
        const int P = (ne + kBucketThreads - 1) / kBucketThreads;
        const int i0 = t * P;
        int loc = 0;
        for (int k = 0; k < P; ++k) {
            const int i = i0 + k;
            if (i < ne) loc += s_cnt[(i & 15) * nb + (i >> 4)];
        }
        int tot;
        int run = block_scan_total<kBucketThreads>(loc, s_wtot, &tot);  // (its barrier orders the reads above before the writes below)
        for (int k = 0; k < P; ++k) {
            const int i = i0 + k;
            if (i < ne) {
                int &c = s_cnt[(i & 15) * nb + (i >> 4)];
                const int v = c;
                c = run;
                run += v;
            }
        }
    }
    __syncthreads();
    if (t < nb) {  // key t's run: from its wave-0 position to the next key's
        const int ks = s_cnt[t], ke = t + 1 < nb ? s_cnt[t + 1] : size;
        const int tile = padded_tile(G, key0 | (unsigned)t);
        if (tile != kInvalidKey)
            tile_bins[tile] = ke > ks ? make_int2((int)(start + ks), (int)(start + ke))
                                      : make_int2(0, 0);
    }
    const bool staged = size <= kStageWords<LB>;
    __syncthreads();
    const uint64_t lt = lanemask_lt();
    for (int j = 0; j < nbatch; ++j) {
        if (nbatch > 1) load(j);
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            const int i0 = s0 + (j * kBatch + q) * kWave;
            if (i0 >= s1) break;  // uniform in the wave
            const bool valid = i0 + lane < s1;
            const int d = (int)(w[q] & lmask);
            const uint64_t vm = __ballot(valid);
            uint32_t plo = (uint32_t)vm, phi = (uint32_t)(vm >> 32);
            for (int bit = 0; bit < lb; ++bit) {  // lanes whose low digit equals d
                const uint32_t x = (uint32_t)__builtin_amdgcn_sbfe(d, bit, 1);
                const uint64_t m = __ballot(x != 0u);
                plo &= ~((uint32_t)m ^ x);
                phi &= ~((uint32_t)(m >> 32) ^ x);
            }
            const uint64_t peers = ((uint64_t)phi << 32) | plo;
            const int r = __popcll(peers & lt);
            const int off = cnt[d];  // the wave's own counter: LDS keeps read-then-write order
            if (valid && r == 0) cnt[d] = off + __popcll(peers);
            if (valid) {
                const int pos = off + r;
                if (staged) {
                    s_stage[pos] = w[q];
                } else {
                    vout[start + pos] = (int)(w[q] >> lb);
                    if (kout) kout[start + pos] = padded_tile(G, key0 | (unsigned)d);
                }
            }
        }
    }
    if (staged) {
        __syncthreads();
        for (int i = t; i < size; i += kBucketThreads) {
            const unsigned x = s_stage[i];
            vout[start + i] = (int)(x >> lb);
            if (kout) kout[start + i] = padded_tile(G, key0 | (x & lmask));
        }
    }
}

struct BinLayout {
    size_t keys_a, vals_a, keys_b, hist, totals, total;
    int bits, passes, nblocks, hstride;  // LSD digit width; hist row stride, a multiple of 4
    bool bucket;     // the bucket path (box rows split by bucket + k_bucket_sort)
    BucketGeom geom; // its padded-key geometry
    int nchunks, bstride;  // its chunks of kSplitThreads Gaussians and their hist row stride
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// The bucket path serves padded keys of up to 18 bits (at most 9 low bits per
// bucket) while the buckets stay small enough for one workgroup each (mean
// capacity below kBucketMeanMax pairs); heavier scenes (e.g. 118M pairs on 2^15 tiles)
// keep the LSD passes, whose every pass spreads over all CUs.  GSV_BINNING=lsd
// or =bucket overrides the choice (bucket only where the key width allows it),
// so that tests can run both paths on one scene; the workspace is the same
// either way (its hist region fits both paths' histograms).  allow_bucket =
// false leaves the bucket path out of the layout altogether.
constexpr int64_t kBucketMeanMax = 40000;  // ~1.1 x the 35,840 words a bucket sort stages

BinLayout bin_layout(int64_t cap, int Tx, int Ty, int Tz, int64_t n, bool allow_bucket = true) {
    BinLayout L{};
    const int64_t n_tiles = (int64_t)Tx * Ty * Tz;
    int bits = 0;
    while (bits < 31 && ((int64_t)1 << bits) < n_tiles) ++bits;
    L.bits = (bits == 17 || bits == 18) ? 9 : 8;
    L.passes = (bits + L.bits - 1) / L.bits;
    // padded keys: xb bits of x, rb bits of the Ty * Tz rows; the top digit
    // takes at most rb bits, so that the low bits hold whole rows
    int xb = 0, rb = 0;
    while (xb < 31 && (1 << xb) < Tx) ++xb;
    while (rb < 31 && ((int64_t)1 << rb) < (int64_t)Ty * Tz) ++rb;
    const int pbits = xb + rb;
    L.geom.Tx = Tx;
    L.geom.Ty = Ty;
    L.geom.rows = Ty * Tz;  // <= n_tiles, checked below 2^31 by the caller
    L.geom.xb = xb;
    // top digit: 8 bits, 9 for 17-bit keys, 10 for 18-bit ones, so that a bucket
    // holds at most 2^8 keys and its sort stages in the 140 KiB LDS variant
    const int want = pbits >= 18 ? 10 : (pbits >= 17 ? 9 : 8);
    L.geom.nbits = rb < want ? rb : want;
    L.geom.lb = pbits - L.geom.nbits;
    // gaussian ids must fit beside the low bits in a word
    const bool allow = allow_bucket && pbits <= 18 && L.geom.lb <= kRadixBitsMax &&
                       n <= ((int64_t)1 << (32 - L.geom.lb));
    const char *force = getenv("GSV_BINNING");
    if (force && strcmp(force, "lsd") == 0) L.bucket = false;
    else if (force && strcmp(force, "bucket") == 0) L.bucket = allow;
    else L.bucket = allow && cap <= ((int64_t)1 << L.geom.nbits) * kBucketMeanMax;
    L.nblocks = (int)((cap + kChunk - 1) / kChunk);
    L.hstride = (imax64(L.nblocks, 1) + 3) / 4 * 4;
    L.nchunks = (int)((n + kSplitThreads - 1) / kSplitThreads);
    L.bstride = (imax64(L.nchunks, 1) + 3) / 4 * 4;
    const size_t arr = align256((size_t)cap * sizeof(int));
    size_t hist_bytes = ((size_t)1 << L.bits) * L.hstride * sizeof(int);
    size_t tot_bytes = ((size_t)1 << L.bits) * sizeof(int);
    if (allow) {
        const size_t bh = ((size_t)1 << L.geom.nbits) * L.bstride * sizeof(int);
        hist_bytes = bh > hist_bytes ? bh : hist_bytes;
        const size_t bt = ((size_t)1 << L.geom.nbits) * sizeof(int);
        tot_bytes = bt > tot_bytes ? bt : tot_bytes;
    }
    size_t off = 0;
    L.keys_a = off; off += arr;
    L.vals_a = off; off += arr;
    L.keys_b = off; off += arr;
    L.hist = off; off += align256(hist_bytes);
    L.totals = off; off += align256(tot_bytes);
    L.total = off;
    return L;
}

// Emission and the LSD passes with B-bit digits, ping-ponging between (ka, va)
// and (kb, vb) so that the last pass ends in (kb, vb); *keys_sorted gets the
// buffer of the sorted keys.
template <int B>
int emit_and_sort(const BinLayout &L, int32_t n, int64_t cap, const int64_t *d_count,
                  const int32_t *tile_min, const int32_t *tile_max, const int32_t *cum, int Tx,
                  int Ty, int64_t T, int *ka, int *va, int *kb, int *vb, int *hist, int *totals,
                  int32_t *tile_bins, hipStream_t s, int **keys_sorted) {
    int *kin = (L.passes % 2 == 0) ? kb : ka;
    int *vin = (L.passes % 2 == 0) ? vb : va;
    hipLaunchKernelGGL(k_emit_chunk<B>, dim3(L.nblocks), dim3(kEmitThreads), 0, s, n, cap,
                       d_count, tile_min, tile_max, cum, Tx, Ty, T, kin, vin, hist, L.hstride, 0,
                       reinterpret_cast<int2 *>(tile_bins));
    if (int st = check_launch()) return st;
    for (int p = 0; p < L.passes; ++p) {
        int *kout = (kin == ka) ? kb : ka;
        int *vout = (vin == va) ? vb : va;
        const int shift = p * B;
        if (p > 0) {
            hipLaunchKernelGGL(k_radix_hist<B>, dim3(L.nblocks), dim3(kSortThreads), 0, s, kin,
                               cap, d_count, shift, hist, L.hstride);
            if (int st = check_launch()) return st;
        }
        hipLaunchKernelGGL(k_digit_scan, dim3(1u << B), dim3(kDigitScanThreads), 0, s, hist,
                           L.nblocks, L.hstride, totals);
        if (int st = check_launch()) return st;
        const int remap = L.nblocks > kRemapChunks ? 1 : 0;
        hipLaunchKernelGGL(k_radix_scatter<B>,
                           dim3((unsigned)(remap ? kXcds * xcd_per(L.nblocks) : L.nblocks)),
                           dim3(kSortThreads), 0, s, kin, vin, kout, vout, cap, d_count, shift,
                           hist, totals, L.nblocks, L.hstride, remap);
        if (int st = check_launch()) return st;
        kin = kout;
        vin = vout;
    }
    *keys_sorted = kin;
    return GSV_OK;
}

// The bucket path's last two launches: the stable split of the box rows into
// buckets of packed words (in ka), then k_bucket_sort into (tiles_out, ids_out)
// and tile_bins.  hist holds the chunks' prefixes per digit, totals the digit
// totals.
template <int Bt>
int split_and_bucket_sort(const BinLayout &L, int32_t n, int64_t cap, const int32_t *tile_min,
                          const int32_t *tile_max, const int32_t *cum, int *ka, const int *hist,
                          const int *totals, int32_t *ids_out, int32_t *tiles_out,
                          int32_t *tile_bins, hipStream_t s) {
    const unsigned blocks = (unsigned)L.nchunks;
    unsigned *words = reinterpret_cast<unsigned *>(ka);
    hipLaunchKernelGGL(k_bucket_split<Bt>, dim3(blocks), dim3(kSplitThreads), 0, s, n, cap,
                       tile_min, tile_max, cum, L.geom, hist, L.bstride, totals, words);
    if (int st = check_launch()) return st;
    // every padded key of [0, 2^(nbits + lb)) lies in one of the 2^nbits buckets
    if (L.geom.lb <= 8)
        hipLaunchKernelGGL(k_bucket_sort<8>, dim3(1u << L.geom.nbits), dim3(kBucketThreads), 0, s,
                           words, tiles_out, ids_out, totals, L.geom, cap,
                           reinterpret_cast<int2 *>(tile_bins));
    else
        hipLaunchKernelGGL(k_bucket_sort<9>, dim3(1u << L.geom.nbits), dim3(kBucketThreads), 0, s,
                           words, tiles_out, ids_out, totals, L.geom, cap,
                           reinterpret_cast<int2 *>(tile_bins));
    return check_launch();
}

// The bucket path: box rows counted per chunk of Gaussians and top digit,
// the prefix over chunks, the stable split of the rows into buckets of packed
// words (in ka), then k_bucket_sort into (tiles_out, ids_out) and tile_bins.
// Four launches; Bt sizes the top digit's LDS arrays (8 or 9 bits).
template <int Bt>
int rows_and_bucket_sort(const BinLayout &L, int32_t n, int64_t cap, const int32_t *tile_min,
                         const int32_t *tile_max, const int32_t *cum, int *ka, int *hist,
                         int *totals, int32_t *ids_out, int32_t *tiles_out, int32_t *tile_bins,
                         hipStream_t s) {
    const unsigned blocks = (unsigned)L.nchunks;
    hipLaunchKernelGGL(k_bucket_hist<Bt>, dim3(blocks), dim3(kSplitThreads), 0, s, n, cap,
                       tile_min, tile_max, cum, L.geom, hist, L.bstride);
    if (int st = check_launch()) return st;
    hipLaunchKernelGGL(k_digit_scan, dim3(1u << L.geom.nbits), dim3(kDigitScanThreads), 0, s,
                       hist, L.nchunks, L.bstride, totals);
    if (int st = check_launch()) return st;
    return split_and_bucket_sort<Bt>(L, n, cap, tile_min, tile_max, cum, ka, hist, totals, ids_out,
                                     tiles_out, tile_bins, s);
}

// tiles_out (optional, 16-byte aligned, cap entries): the sorted keys, i.e. the
// tile of each sorted pair, written by the last pass in place of a workspace
// buffer.
int bin_and_sort(int32_t n, int64_t cap, const int64_t *d_count, const int32_t *tile_min,
                 const int32_t *tile_max, const int32_t *cum, int32_t D, int32_t H, int32_t W,
                 void *workspace, size_t workspace_bytes, int32_t *ids_out, int32_t *tile_bins,
                 int32_t *tiles_out, hipStream_t s, bool allow_bucket = true) {
    if (n < 0 || D <= 0 || H <= 0 || W <= 0 || !tile_bins) return GSV_ERR_INVALID_ARGUMENT;
    if (cap > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    const int64_t T = (int64_t)Tx * Ty * Tz;
    if (T > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    if (cap <= 0 || n == 0) return fill_zero_u32(tile_bins, 2 * T, s);
    if (!tile_min || !tile_max || !cum || !ids_out || !workspace) return GSV_ERR_INVALID_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(ids_out) & 15) != 0) return GSV_ERR_INVALID_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(tiles_out) & 15) != 0) return GSV_ERR_INVALID_ARGUMENT;
    const BinLayout L = bin_layout(cap, Tx, Ty, Tz, n, allow_bucket);
    if (workspace_bytes < L.total + 256) return GSV_ERR_WORKSPACE_TOO_SMALL;
    char *ws = static_cast<char *>(workspace);
    ws += (256 - (reinterpret_cast<uintptr_t>(ws) & 255)) & 255;  // 16-byte vector access
    int *ka = reinterpret_cast<int *>(ws + L.keys_a);
    int *va = reinterpret_cast<int *>(ws + L.vals_a);
    int *hist = reinterpret_cast<int *>(ws + L.hist);
    int *totals = reinterpret_cast<int *>(ws + L.totals);
    if (L.bucket) {  // works from cum and the capacity alone: no pair count needed
        if (L.geom.nbits == 10)
            return rows_and_bucket_sort<10>(L, n, cap, tile_min, tile_max, cum, ka, hist, totals,
                                            ids_out, tiles_out, tile_bins, s);
        return L.geom.nbits == 9
                   ? rows_and_bucket_sort<9>(L, n, cap, tile_min, tile_max, cum, ka, hist, totals,
                                             ids_out, tiles_out, tile_bins, s)
                   : rows_and_bucket_sort<8>(L, n, cap, tile_min, tile_max, cum, ka, hist, totals,
                                             ids_out, tiles_out, tile_bins, s);
    }
    int *kb = tiles_out ? tiles_out : reinterpret_cast<int *>(ws + L.keys_b);
    int *vb = ids_out;
    int *keys_sorted = nullptr;
    const int st = L.bits == 9 ? emit_and_sort<9>(L, n, cap, d_count, tile_min, tile_max, cum, Tx,
                                                  Ty, T, ka, va, kb, vb, hist, totals, tile_bins,
                                                  s, &keys_sorted)
                               : emit_and_sort<8>(L, n, cap, d_count, tile_min, tile_max, cum, Tx,
                                                  Ty, T, ka, va, kb, vb, hist, totals, tile_bins,
                                                  s, &keys_sorted);
    if (st) return st;
    const int64_t threads = (cap + kEdgeItems - 1) / kEdgeItems;
    hipLaunchKernelGGL(k_tile_edges, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       keys_sorted, cap, d_count, T, reinterpret_cast<int2 *>(tile_bins));
    return check_launch();
}

// The prefix sum of num_tiles_hit (cum, *total_out, *total_host_dev) and the
// binning with the count left on the device, in one call.  The workspace holds
// the scan's block sums (align256(scan_workspace_bytes(n)) bytes) and then the
// binning's.  On the bucket path with a direct scan (at most kDirectBlocks
// blocks) the bucket counts and their prefix ride on the scan's launches
// (k_sums_hist, k_apply_digits); otherwise the scan and bin_and_sort run one
// after the other.
size_t cumsum_scan_bytes(int64_t n) { return align256(scan_workspace_bytes(n)); }

template <int Bt>
int fused_bucket_path(const BinLayout &L, int32_t n, int64_t cap, const int32_t *nth,
                      const int32_t *tile_min, const int32_t *tile_max, int32_t *cum,
                      int64_t *total_out, int64_t *total_host_dev, int32_t *part, int *ka,
                      int *hist, int *totals, int32_t *ids_out, int32_t *tile_bins,
                      int32_t *tiles_out, hipStream_t s) {
    const int nb_scan = (int)((n + scan_detail::kTile - 1) / scan_detail::kTile);
    hipLaunchKernelGGL(k_sums_hist<Bt>, dim3((unsigned)(nb_scan + L.nchunks)), dim3(kSplitThreads),
                       0, s, nth, n, nb_scan, part, tile_min, tile_max, L.geom, hist, L.bstride);
    if (int st = check_launch()) return st;
    hipLaunchKernelGGL(k_apply_digits, dim3((unsigned)(nb_scan + (1 << L.geom.nbits))),
                       dim3(kSplitThreads), 0, s, nth, cum, n, nb_scan, part, total_out,
                       total_host_dev, hist, L.nchunks, L.bstride, totals);
    if (int st = check_launch()) return st;
    return split_and_bucket_sort<Bt>(L, n, cap, tile_min, tile_max, cum, ka, hist, totals, ids_out,
                                     tiles_out, tile_bins, s);
}

int cumsum_bin_and_sort(int32_t n, int64_t cap, const int32_t *nth, const int32_t *tile_min,
                        const int32_t *tile_max, int32_t D, int32_t H, int32_t W, int32_t *cum,
                        int64_t *total_out, int64_t *total_host_dev, void *workspace,
                        size_t workspace_bytes, int32_t *ids_out, int32_t *tile_bins,
                        int32_t *tiles_out, hipStream_t s) {
    if (n < 0 || D <= 0 || H <= 0 || W <= 0 || !tile_bins || !total_out || !workspace)
        return GSV_ERR_INVALID_ARGUMENT;
    if (n > 0 && (!nth || !cum)) return GSV_ERR_INVALID_ARGUMENT;
    if (cap > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    if ((int64_t)Tx * Ty * Tz > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const size_t scan_bytes = cumsum_scan_bytes(n);
    if (workspace_bytes < scan_bytes) return GSV_ERR_WORKSPACE_TOO_SMALL;
    char *bin_ws = static_cast<char *>(workspace) + scan_bytes;
    const size_t bin_bytes = workspace_bytes - scan_bytes;
    const int64_t nb_scan = ((int64_t)n + scan_detail::kTile - 1) / scan_detail::kTile;
    bool fused = cap > 0 && n > 0 && nb_scan <= scan_detail::kDirectBlocks && tile_min &&
                 tile_max && ids_out;
    BinLayout L{};
    if (fused) {
        L = bin_layout(cap, Tx, Ty, Tz, n);
        fused = L.bucket;
    }
    if (!fused) {
        if (int st = scan_i32(nth, cum, n, true, total_out, total_host_dev, workspace, scan_bytes, s))
            return st;
        return bin_and_sort(n, cap, total_out, tile_min, tile_max, cum, D, H, W, bin_ws, bin_bytes,
                            ids_out, tile_bins, tiles_out, s);
    }
    // bin_and_sort's checks for the bucket path
    if ((reinterpret_cast<uintptr_t>(ids_out) & 15) != 0) return GSV_ERR_INVALID_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(tiles_out) & 15) != 0) return GSV_ERR_INVALID_ARGUMENT;
    if (bin_bytes < L.total + 256) return GSV_ERR_WORKSPACE_TOO_SMALL;
    char *ws = bin_ws + ((256 - (reinterpret_cast<uintptr_t>(bin_ws) & 255)) & 255);
    int32_t *part = static_cast<int32_t *>(workspace);
    int *ka = reinterpret_cast<int *>(ws + L.keys_a);
    int *hist = reinterpret_cast<int *>(ws + L.hist);
    int *totals = reinterpret_cast<int *>(ws + L.totals);
    switch (L.geom.nbits) {
        case 10:
            return fused_bucket_path<10>(L, n, cap, nth, tile_min, tile_max, cum, total_out,
                                         total_host_dev, part, ka, hist, totals, ids_out,
                                         tile_bins, tiles_out, s);
        case 9:
            return fused_bucket_path<9>(L, n, cap, nth, tile_min, tile_max, cum, total_out,
                                        total_host_dev, part, ka, hist, totals, ids_out, tile_bins,
                                        tiles_out, s);
        default:
            return fused_bucket_path<8>(L, n, cap, nth, tile_min, tile_max, cum, total_out,
                                        total_host_dev, part, ka, hist, totals, ids_out, tile_bins,
                                        tiles_out, s);
    }
}

// ---------------------------------------------------- allocation-free entry --

// The workspace of gsv_bin_and_sort_noalloc: bin_layout() at the largest
// supported pair count and the widest digit, plus the 256 bytes of alignment
// slack bin_and_sort() takes.  One copy per GPU, allocated when the library's
// code object is loaded on that GPU.
constexpr int64_t kNoAllocMaxPairs = GSV_NOALLOC_MAX_INTERSECTIONS;
constexpr size_t kNoAllocArr = ((size_t)kNoAllocMaxPairs * sizeof(int) + 255) / 256 * 256;
constexpr size_t kNoAllocHistStride = ((kNoAllocMaxPairs + kChunk - 1) / kChunk + 3) / 4 * 4;
constexpr size_t kNoAllocScratchBytes =
    3 * kNoAllocArr + ((size_t)kRadixBinsMax * kNoAllocHistStride * sizeof(int) + 255) / 256 * 256 +
    ((size_t)kRadixBinsMax * sizeof(int) + 255) / 256 * 256 + 256;
static_assert(kNoAllocScratchBytes == 52431104, "the size gsvox.h states");

}  // namespace
}  // namespace gsv

// In host code this name is only a handle for hipGetSymbolAddress: each GPU
// holds its own copy at its own address (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[gsv::kNoAllocScratchBytes];

namespace gsv {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch[kMaxDevices];  // device address of `scratch` on each GPU, once looked up

// The current device's copy of `scratch`, looked up once per device with that
// device current.
int noalloc_scratch(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return record_hip_error(e);
    if (dev < 0 || dev >= kMaxDevices) return GSV_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return record_hip_error(e);
        if (p == nullptr) return GSV_ERR_HIP;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return GSV_OK;
}

}  // namespace
}  // namespace gsv

using namespace gsv;

extern "C" int gsv_bin_workspace_bytes(int32_t n, int64_t num_intersects, int32_t D, int32_t H,
                                       int32_t W, size_t *bytes) {
    if (!bytes || n < 0 || D <= 0 || H <= 0 || W <= 0) return GSV_ERR_INVALID_ARGUMENT;
    if (num_intersects > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    if ((int64_t)Tx * Ty * Tz > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const BinLayout L = bin_layout(num_intersects > 0 ? num_intersects : 0, Tx, Ty, Tz, n);
    *bytes = L.total + 256;
    return GSV_OK;
}

extern "C" int gsv_bin_and_sort(int32_t n, int64_t num_intersects, const int32_t *tile_min,
                                const int32_t *tile_max, const int32_t *cum_tiles_hit, int32_t D,
                                int32_t H, int32_t W, void *workspace, size_t workspace_bytes,
                                int32_t *gaussian_ids_sorted, int32_t *tile_bins,
                                int32_t *tiles_sorted, void *stream) {
    return bin_and_sort(n, num_intersects, nullptr, tile_min, tile_max, cum_tiles_hit, D, H, W,
                        workspace, workspace_bytes, gaussian_ids_sorted, tile_bins, tiles_sorted,
                        as_stream(stream));
}

extern "C" int gsv_bin_and_sort_device_count(int32_t n, int64_t capacity,
                                             const int64_t *num_intersects_dev,
                                             const int32_t *tile_min, const int32_t *tile_max,
                                             const int32_t *cum_tiles_hit, int32_t D, int32_t H,
                                             int32_t W, void *workspace, size_t workspace_bytes,
                                             int32_t *gaussian_ids_sorted, int32_t *tile_bins,
                                             int32_t *tiles_sorted, void *stream) {
    if (!num_intersects_dev) return GSV_ERR_INVALID_ARGUMENT;
    return bin_and_sort(n, capacity, num_intersects_dev, tile_min, tile_max, cum_tiles_hit, D, H,
                        W, workspace, workspace_bytes, gaussian_ids_sorted, tile_bins,
                        tiles_sorted, as_stream(stream));
}

extern "C" int gsv_cumsum_bin_workspace_bytes(int32_t n, int64_t capacity, int32_t D, int32_t H,
                                              int32_t W, size_t *bytes) {
    if (!bytes) return GSV_ERR_INVALID_ARGUMENT;
    size_t bin = 0;
    if (int st = gsv_bin_workspace_bytes(n, capacity, D, H, W, &bin)) return st;
    *bytes = cumsum_scan_bytes(n) + bin;
    return GSV_OK;
}

extern "C" int gsv_cumsum_bin_and_sort_device_count(
    int32_t n, int64_t capacity, const int32_t *num_tiles_hit, const int32_t *tile_min,
    const int32_t *tile_max, int32_t D, int32_t H, int32_t W, int32_t *cum_tiles_hit,
    int64_t *total_out, int64_t *total_host, void *workspace, size_t workspace_bytes,
    int32_t *gaussian_ids_sorted, int32_t *tile_bins, int32_t *tiles_sorted, void *stream) {
    int64_t *host_dev = nullptr;
    if (int st = pinned_int64_device_ptr(total_host, &host_dev)) return st;
    return cumsum_bin_and_sort(n, capacity, num_tiles_hit, tile_min, tile_max, D, H, W,
                               cum_tiles_hit, total_out, host_dev, workspace, workspace_bytes,
                               gaussian_ids_sorted, tile_bins, tiles_sorted, as_stream(stream));
}

extern "C" int gsv_bin_and_sort_noalloc(int32_t n, int64_t num_intersects,
                                        const int32_t *tile_min, const int32_t *tile_max,
                                        const int32_t *cum_tiles_hit, int32_t D, int32_t H,
                                        int32_t W, int32_t *gaussian_ids_sorted,
                                        int32_t *tile_bins, int32_t *tiles_sorted, void *stream) {
    if (num_intersects > kNoAllocMaxPairs) return GSV_ERR_SCRATCH_TOO_SMALL;
    if (n < 0 || D <= 0 || H <= 0 || W <= 0) return GSV_ERR_INVALID_ARGUMENT;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    if ((int64_t)Tx * Ty * Tz > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    // the bucket path's histogram grows with the Gaussian count: where it would
    // not fit the scratch array, the LSD passes (sized by the pair count) serve
    const int64_t np = num_intersects > 0 ? num_intersects : 0;
    bool bucket = bin_layout(np, Tx, Ty, Tz, n).total + 256 <= kNoAllocScratchBytes;
    if (!bucket && bin_layout(np, Tx, Ty, Tz, n, false).total + 256 > kNoAllocScratchBytes)
        return GSV_ERR_SCRATCH_TOO_SMALL;
    void *ws = nullptr;
    if (int st = noalloc_scratch(&ws)) return st;
    return bin_and_sort(n, num_intersects, nullptr, tile_min, tile_max, cum_tiles_hit, D, H, W,
                        ws, kNoAllocScratchBytes, gaussian_ids_sorted, tile_bins, tiles_sorted,
                        as_stream(stream), bucket);
}
