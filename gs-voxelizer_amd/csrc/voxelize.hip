// voxelize.hip — forward and backward Gaussian voxelization for gfx950.
//
// Reference kernels: voxelize_forward (gs_voxelizer/cuda/voxelize.cu:39-164),
// voxelize_backward (170-366) and voxelize_backward_per_gaussian (368-610),
// launched by bindings.cu:362-781.  Semantics kept: 8x8x8 voxel tiles, each
// voxel sums every Gaussian of its tile's list, voxel centres at index + 0.5,
// the gates `sigma > 0 || nan || inf` and `alpha * mean(I) < 1e-6`.
//
// How the work maps to CDNA4 (not the reference's CUDA mapping):
//  * exp is evaluated as exp2 on a log2-scaled quadratic form, and both gates
//    collapse into one compare |s| <= h:  with sigma2 = sigma*log2(e) and
//    t2 = log2(1e-6 / mean), a Gaussian contributes iff t2 <= sigma2 <= 0.
//    Writing s = sigma2 - t2/2, h = -t2/2 makes that |s| <= h, and the factor
//    2^(t2/2) is folded into the intensities (forward) or the final gradient
//    scale (backward).
//  * Gate-free evaluation.  v_exp_f32 returns exactly 0 for every result below
//    2^-126 (it produces no denormals) and exactly 2^-126 at -126.  With
//    off = -(t2 + 126), rounded once, exp2(sigma2 + off) is therefore nonzero
//    iff sigma2 >= t2 (up to that rounding), and 2^-off restores the
//    magnitude.  For a finite positive-definite conic sigma2 <= 0 holds
//    everywhere (up to rounding), so both gates cost no instruction at all.
//    Gaussians outside that domain (indefinite or non-finite conic, mean
//    beyond 2^60 * 1e-6, intensities far above the mean) take the exact
//    |s| <= h path.
//  * This file is compiled in binary32 flush-to-zero mode
//    (-fgpu-flush-denormals-to-zero): v_mul_f32 then also returns 0 below
//    2^-126, so both kernels form most of a row's exp2 values as products
//    with the same gate: two or three v_exp_f32 per 8-voxel row instead of
//    eight.  A v_exp_f32 issues at about half an FMA's rate (0.106 against
//    0.222 wave64 instructions per SIMD-cycle on a throughput probe) and does
//    not overlap the other VALU work, so the eight-exp row spent about as much
//    time in them as in its 28 other instructions.  Elsewhere the kernels
//    keep every binary32 value they rely on in
//    the normal range (the backward's power-of-two staging of vol_grad), so
//    the mode changes no result beyond denormal magnitudes.
//  * Along a voxel row (fixed y, z) the quadratic form is
//    s(dx) = R0 + dx*(R1 + A2*dx): two FMAs per voxel once R0, R1 are set up.
//  * Forward: one 64-lane wave per tile, lane = one x-row of 8 voxels.  Per
//    batch of 64 Gaussians each lane prepares one Gaussian's row constants into
//    LDS; the wave then walks the live ones, reading each record with a
//    uniform-address (broadcast) LDS read, so no VALU slot is spent on
//    broadcasting.
//  * Backward: one wave per bucket of 64 (tile, Gaussian) pairs, lane = one
//    Gaussian; the tile's vol_grad is staged once in LDS and read row by row
//    with broadcast reads.  Each lane accumulates its Gaussian's moments
//    sum(w), sum(w*d), sum(w*d*d^T) in registers and turns them into the conic
//    and mean gradients once, then issues one atomic per output component.
//  * Tile culling: a Gaussian whose gate ellipsoid sigma >= ln(1e-6/mean)
//    (a bounded ellipsoid for positive-definite conics) misses every voxel
//    centre of a tile contributes exactly nothing there in the reference; such
//    (tile, Gaussian) pairs are skipped with a conservative axis-aligned test.
#include <float.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "gsv_device.h"
#include "gsv_scan.h"

namespace gsv {
namespace {

constexpr float kLog2e = 1.44269504088896341f;
constexpr float kLn2 = 0.693147180559945309f;
constexpr float kLog2MinContrib = -19.9315685693241741f;  // log2(1e-6)

constexpr float kExpFlush = 126.0f;     // v_exp_f32 results below 2^-126 are 0

// The forward at C = 1 accumulates I * alpha / kAccUnit, kAccUnit = fl(1e-6) * 2^126:
// a term then falls below 2^-126, and a product that forms it is flushed to 0,
// exactly when I * alpha < fl(1e-6), the reference's gate.  The chained rows fold
// the weight I * 2^-off / kAccUnit (1 up to the rounding of off) into their
// per-Gaussian factors, so each voxel's gated product is added with a
// two-operand v_add_f32 instead of a three-operand FMA against the weight; the
// other paths scale their weights alike, and the epilogue multiplies once.
constexpr float kAccUnit = 1e-6f * 0x1p126f;
constexpr float kInvAccUnit = (float)(1.0 / (double)kAccUnit);  // rounded once: ~1e-7 overall
constexpr float kDeadOffset = -1000.0f;  // exponent offset that zeroes a lane
constexpr float kFwdFastConicMax = 4096.0f;  // largest conic diagonal of the forward's gate-free rows

struct Gate {
    float shift;   // exact path: s = sigma2 - shift
    float half;    // exact path: contributes iff |s| <= half
    float scale;   // exact path: 2^shift
    float off;     // gate-free path: a = exp2(sigma2 + off)
    float fscale;  // gate-free path: 2^-off
    float t2;      // log2(1e-6 / mean), or 0 when unbounded
    bool live;
    bool bounded;
};

// Gate constants from the mean intensity (voxelize.cu:138-148).
__device__ __forceinline__ Gate make_gate(float mean) {
    Gate g;
    g.off = kDeadOffset;
    g.fscale = 0.f;
    if (mean > 0.f && mean <= FLT_MAX) {
        const float t2 = kLog2MinContrib - __log2f(mean);
        g.t2 = t2;
        g.shift = 0.5f * t2;
        g.half = -0.5f * t2;
        g.scale = __builtin_amdgcn_exp2f(g.shift);  // shift >= -75 for a finite mean: a normal result
        g.live = t2 <= 0.f;  // mean < 1e-6: alpha <= 1 can never reach the threshold
        g.bounded = true;
        if (g.live && t2 >= -60.f) {
            g.off = -(t2 + kExpFlush);
            g.fscale = __builtin_amdgcn_exp2f(-g.off);  // of the rounded offset (66..126), so the two cancel
        }
    } else if (mean > 0.f || mean != mean) {
        // +inf or NaN mean: the reference's `alpha * mean < 1e-6` never holds,
        // every finite sigma <= 0 contributes I * alpha.
        g.t2 = 0.f;
        g.shift = 0.f;
        g.half = __builtin_inff();
        g.scale = 1.f;
        g.live = true;
        g.bounded = false;
    } else {
        g.t2 = 0.f; g.shift = 0.f; g.half = -1.f; g.scale = 0.f;
        g.live = false;  // mean <= 0: alpha * mean < 1e-6 always
        g.bounded = false;
    }
    return g;
}

// Whether a live Gaussian may use the gate-free evaluation: bounded gate with
// t2 >= -60, intensities whose weights I * 2^-off stay below 2^120, a finite
// centre and a finite positive-definite conic (Sylvester's criterion), so that
// sigma2 <= 0 up to rounding and every product in the kernels stays finite.
__device__ __forceinline__ bool gate_free_ok(const Gate &g, float max_abs_i, float mx, float my,
                                             float mz, float a, float b, float c, float d, float e,
                                             float f) {
    if (!g.live || !g.bounded || !(g.fscale > 0.f)) return false;
    if (!(max_abs_i * g.fscale <= 0x1p120f)) return false;
    if (!__builtin_isfinite(mx + my + mz) || !__builtin_isfinite(a + b + c + d + e + f))
        return false;
    const float det = a * (d * f - e * e) - b * (b * f - c * e) + c * (b * e - c * d);
    return a > 0.f && a * d - b * b > 0.f && det > 0.f;
}

// Conservative test: can the ellipsoid {d^T Q d <= K^2}, K^2 = 2 ln(mean*1e6),
// centred at (mx,my,mz), contain a point of the box [lo, hi]?  Only answers
// "no" for a positive-definite Q; margins cover binary32 rounding of the gate.
// Two separating-axis tests: the coordinate axes (the ellipsoid's bounding
// box), then the axis n = Q (c - mu) through the box centre c.  Along n the
// ellipsoid spans n.mu +- K sqrt(n^T Q^-1 n) = n.mu +- K sqrt(m) and the box
// n.c +- sum |n_i| e_i, with m = (c - mu)^T Q (c - mu) = n.(c - mu), so they
// are apart when m - K sqrt(m) > sum |n_i| e_i.  The reference's 3-sigma tile
// boxes make the first test pass for every pair they list; the second finds
// ~90% of the pairs none of whose voxel centres passes the gate (~12% of all
// pairs on uniform scenes: small Gaussians at the corners of their boxes).
__device__ __forceinline__ bool may_touch(float mx, float my, float mz, float a, float b, float c,
                                          float d, float e, float f, float t2, float xlo,
                                          float xhi, float ylo, float yhi, float zlo, float zhi) {
    const float cfx = d * f - e * e, cfy = a * f - c * c, cfz = a * d - b * b;
    const float det = a * cfx - b * (b * f - c * e) + c * (b * e - c * d);
    if (!(a > 0.f && cfz > 0.f && det > 0.f)) return true;
    // In flush-to-zero mode the reciprocal of det >= 2^126 is 0, which would
    // shrink the half-widths below to 0.01: keep such (very thin) Gaussians.
    if (!(det < 0x1p125f)) return true;
    const float k2 = -2.0f * kLn2 * t2;
    const float inv = __builtin_amdgcn_rcpf(det);
    const float hx = __builtin_amdgcn_sqrtf(k2 * cfx * inv) * 1.001f + 0.01f;
    const float hy = __builtin_amdgcn_sqrtf(k2 * cfy * inv) * 1.001f + 0.01f;
    const float hz = __builtin_amdgcn_sqrtf(k2 * cfz * inv) * 1.001f + 0.01f;
    const bool miss = (mx + hx < xlo) || (mx - hx > xhi) || (my + hy < ylo) || (my - hy > yhi) ||
                      (mz + hz < zlo) || (mz - hz > zhi);
    if (miss) return false;
    // m and r in binary64: m can cancel for an elongated conic (its binary32
    // error bound is relative to |d|^T |Q| |d|, not to m)
    const float ex = 0.5f * (xhi - xlo), ey = 0.5f * (yhi - ylo), ez = 0.5f * (zhi - zlo);
    const double dx = (xlo + ex) - mx, dy = (ylo + ey) - my, dz = (zlo + ez) - mz;
    const double nx = (double)a * dx + (double)b * dy + (double)c * dz;
    const double ny = (double)b * dx + (double)d * dy + (double)e * dz;
    const double nz = (double)c * dx + (double)e * dy + (double)f * dz;
    const float m = (float)(dx * nx + dy * ny + dz * nz);
    const float r = (float)(fabs(nx) * ex + fabs(ny) * ey + fabs(nz) * ez);
    const float K = __builtin_amdgcn_sqrtf(k2) * 1.001f + 0.01f, sm = __builtin_amdgcn_sqrtf(m);
    return !(sm * (sm - K) > r * 1.001f + 0.01f);  // NaN anywhere -> comparisons false -> keep
}

// x + y, never contracted with a product that feeds it: the operand is a
// separately rounded (and, below 2^-126, flushed) binary32 product.
__device__ __forceinline__ float add_nc(float x, float y) {
#pragma clang fp contract(off)
    return x + y;
}

__host__ __device__ inline bool aligned_to(const void *p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

struct TileGeom {
    int x0, y0, z0;
    float xlo, xhi, ylo, yhi, zlo, zhi;  // voxel-centre box of the tile's inside voxels
};

// Tile counts are below 2^31 (checked on the host), so 32-bit division serves.
__device__ __forceinline__ TileGeom tile_geom(int tile, int Tx, int Ty, int D, int H, int W) {
    TileGeom t;
    const unsigned q = (unsigned)tile / (unsigned)Tx;
    const int tx = (int)((unsigned)tile - q * (unsigned)Tx);
    const int ty = (int)(q % (unsigned)Ty), tz = (int)(q / (unsigned)Ty);
    t.x0 = tx * GSV_TILE; t.y0 = ty * GSV_TILE; t.z0 = tz * GSV_TILE;
    t.xlo = (float)t.x0 + 0.5f; t.xhi = (float)min(t.x0 + GSV_TILE - 1, W - 1) + 0.5f;
    t.ylo = (float)t.y0 + 0.5f; t.yhi = (float)min(t.y0 + GSV_TILE - 1, H - 1) + 0.5f;
    t.zlo = (float)t.z0 + 0.5f; t.zhi = (float)min(t.z0 + GSV_TILE - 1, D - 1) + 0.5f;
    return t;
}

// The same from a per-lane tile id, with the two divisions as multiply-shifts.
__device__ __forceinline__ TileGeom tile_geom(int tile, FastDiv fx, int Tx, FastDiv fy, int Ty,
                                              int D, int H, int W) {
    TileGeom t;
    const unsigned q = fastdiv((unsigned)tile, fx);
    const int tx = (int)((unsigned)tile - q * (unsigned)Tx);
    const unsigned tz = fastdiv(q, fy);
    const int ty = (int)(q - tz * (unsigned)Ty);
    t.x0 = tx * GSV_TILE; t.y0 = ty * GSV_TILE; t.z0 = (int)tz * GSV_TILE;
    t.xlo = (float)t.x0 + 0.5f; t.xhi = (float)min(t.x0 + GSV_TILE - 1, W - 1) + 0.5f;
    t.ylo = (float)t.y0 + 0.5f; t.yhi = (float)min(t.y0 + GSV_TILE - 1, H - 1) + 0.5f;
    t.zlo = (float)t.z0 + 0.5f; t.zhi = (float)min(t.z0 + GSV_TILE - 1, D - 1) + 0.5f;
    return t;
}

// ---------------------------------------------------------------- forward --

// Fused L1: the forward stores sgn(volume - target) per element as one byte
// for the backward, which then reads 1 byte per element instead of the volume
// and the target.  An unordered difference (a NaN volume or target element)
// stores 0: torch's sign of NaN is 0, so its l1_loss backward passes
// grad * 0 there (NaN only when grad itself is not finite, as here).
// The sign is that of v - t in IEEE arithmetic with denormals (torch's), decided
// on the bit patterns: this file runs in binary32 flush-to-zero mode, where a
// denormal operand would read as 0.  For non-NaN v, t, IEEE v - t is positive
// iff v > t (a difference of distinct floats is never rounded to 0 with
// gradual underflow), and inf - inf is NaN, sign 0, as for equal keys.
__device__ __forceinline__ int order_key(float x) {  // monotone in x; -0 and +0 alike
    const int b = __float_as_int(x);
    return b >= 0 ? b : -(b & 0x7fffffff);
}
__device__ __forceinline__ int8_t l1_sign(float v, float t) {
    if (v != v || t != t) return 0;
    const int kv = order_key(v), kt = order_key(t);
    return kv > kt ? 1 : (kv < kt ? -1 : 0);
}

// float4 slots of one prepared Gaussian record: 13 + C floats (gate-free
// layout) or 12 + C (exact layout).
template <int C>
constexpr int kRecF4 = (13 + C + 3) / 4;

// Six waves per SIMD at C = 1 (78 VGPRs, no spills; 3 us faster at cfg3 than
// five); more channels would spill at six.
template <int C>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(C == 1 ? 6 : 1, 8))) void k_vox_fwd(
    int D, int H, int W, int Tx, int Ty, int64_t T, int n, int n_isect,
    const int *__restrict__ ids, const int2 *__restrict__ bins, const float4 *__restrict__ pos_radii,
    const float2 *__restrict__ conics, const float *__restrict__ intens, float *__restrict__ vol,
    const float *__restrict__ target, float *__restrict__ tile_loss, int8_t *__restrict__ sgn,
    uint8_t *__restrict__ pair_live, uint64_t *__restrict__ wave_rec, int wave_cap) {
    __shared__ float4 s_rec[kWave][kRecF4<C>];
    const int64_t tile = xcd_runs(blockIdx.x);
    if (tile >= T) return;
    const int lane = threadIdx.x;
    const bool timeline = wave_rec != nullptr && (int64_t)blockIdx.x < wave_cap;
    if (timeline && lane == 0) {
        wave_rec[3 * (int64_t)blockIdx.x] = wall_clock64();
        wave_rec[3 * (int64_t)blockIdx.x + 2] = (uint64_t)tile;
    }
    const TileGeom tg = tile_geom((int)tile, Tx, Ty, D, H, W);
    const float py = (float)(lane & 7) - 3.5f, pz = (float)(lane >> 3) - 3.5f;  // centred, tile-local
    const float py2 = py * py, pyz = py * pz, pz2 = pz * pz;                      // exact
    int2 range = bins[tile];
    range.x = max(range.x, 0);
    range.y = min(range.y, n_isect);  // never index past the id array

    float acc[GSV_TILE][C];
#pragma unroll
    for (int u = 0; u < GSV_TILE; ++u)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[u][c] = 0.f;

    for (int b0 = range.x; b0 < range.y; b0 += kWave) {
        const int idx = b0 + lane;
        bool live = false, fast = false, chain = false, one_way = false;
        if (idx < range.y) {
            const int g = ids[idx];
            if ((unsigned)g < (unsigned)n) {
                const float4 p = pos_radii[g];
                const float2 c01 = conics[3 * g], c23 = conics[3 * g + 1], c45 = conics[3 * g + 2];
                float I[C], mean = 0.f, max_abs = 0.f;
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    I[c] = intens[(size_t)g * C + c];
                    mean += I[c];
                    max_abs = fmaxf(max_abs, fabsf(I[c]));
                }
                mean /= (float)C;
                const Gate gt = make_gate(mean);
                live = gt.live;
                if (live && gt.bounded)
                    live = may_touch(p.x, p.y, p.z, c01.x, c01.y, c23.x, c23.y, c45.x, c45.y, gt.t2,
                                     tg.xlo, tg.xhi, tg.ylo, tg.yhi, tg.zlo, tg.zhi);
                if (live) {
                    // the gate-free rows expand the form about the tile centre, whose
                    // terms grow with the conic (~12 |q| at the tile's edge) and cancel
                    // near the Gaussian's centre: conics above kFwdFastConicMax (axes
                    // below 1/64 voxel) take the exact path's direct form instead
                    fast = gate_free_ok(gt, max_abs, p.x, p.y, p.z, c01.x, c01.y, c23.x, c23.y,
                                        c45.x, c45.y) &&
                           fmaxf(c01.x, fmaxf(c23.y, c45.y)) <= kFwdFastConicMax;
                    // centred offsets: delta = c - p', p' = local index - 3.5
                    const float cx = p.x - (float)tg.x0 - 4.0f;
                    const float cy = p.y - (float)tg.y0 - 4.0f, cz = p.z - (float)tg.z0 - 4.0f;
                    const float A2 = -0.5f * kLog2e * c01.x;
                    const float4 q1 = make_float4(-kLog2e * c01.y, -kLog2e * c23.x,
                                                  -0.5f * kLog2e * c23.y, -kLog2e * c45.x);
                    const float F = -0.5f * kLog2e * c45.y;
                    float rec[4 * kRecF4<C>];
                    if (fast) {
                        // The form about the tile centre, in the lane's row offsets
                        // (py, pz):  s(u) = T0 - T1 uc + A2 uc^2 + off with
                        //   T1 = t1 - B py - C pz,
                        //   T0 = t0 + ty py + tz pz + D py^2 + E py pz + F pz^2,
                        // t0 = the form at the tile centre, ty/tz its y/z slopes there.
                        // Formed in binary64 and rounded once.
                        // (t1, -B, -C, t0 | ty, tz, D, E | F, Q0, Q1, Q2 | Q3, I*2^-off ...),
                        // Q_k = A2 * uc_k^2 + off for the four |uc| = 0.5, 1.5, 2.5, 3.5
                        const double X = cx, Y = cy, Z = cz;
                        const double a2 = A2, bb = q1.x, cc = q1.y, dd = q1.z, ee = q1.w, ff = F;
                        rec[0] = (float)(2.0 * a2 * X + bb * Y + cc * Z);
                        rec[1] = -q1.x; rec[2] = -q1.y;
                        const double t0 = X * (a2 * X + bb * Y + cc * Z) + Y * (dd * Y + ee * Z) +
                                          ff * Z * Z;
                        const double ty = -(bb * X + 2.0 * dd * Y + ee * Z);
                        const double tz = -(cc * X + ee * Y + 2.0 * ff * Z);
                        rec[6] = q1.z; rec[7] = q1.w;
                        rec[8] = F;
                        // Chained rows (the first two loops below) split s(u) into
                        //   E(uc) = T0 + off + K - T1 uc   and   G(uc) = A2 uc^2 - K
                        // and form 2^E by products: from uc = -3.5 to +3.5 (one-way
                        // chain, span 7) or from uc = +0.5 outwards both ways (its
                        // first step left gives uc = -0.5; span 4).  With
                        // M >= |T1| on every row of the tile and an integer
                        // K >= span * M + 2, K + 12.25 |A2| <= 120 (K is the largest
                        // such integer: it brings the exp2 arguments of the passing
                        // voxels nearest to 0, where their rounding costs least):
                        //  - every 2^G is a normal number (G >= -120);
                        //  - 2^E <= 2^(-66 + 12.25 |A2| + K) < 2^54 (s <= off <= -66):
                        //    no overflow on any row, live or not;
                        //  - at a voxel with s >= -126, E >= -126 + K, and E is linear
                        //    in uc, so every product of the chain up to it is at
                        //    least 2^(-126 + K - span * M) > 2^-126: no factor is
                        //    flushed early, and a product flushes only where s < -126.
                        // The record's (t0, ty, tz) then hold the anchor's exponent,
                        // E at uc = -3.5 or +0.5: T0 - uc T1 in the same polynomial.
                        const float bound_t1 =
                            (fabsf(rec[0]) + 3.5f * (fabsf(rec[1]) + fabsf(rec[2]))) * 1.001f;
                        const float span_g = 12.25f * fabsf(A2);
                        const float K = floorf(120.0f - span_g);
                        one_way = ceilf(7.0f * bound_t1) + 2.0f <= K;
                        chain = one_way || ceilf(4.0f * bound_t1) + 2.0f <= K;
                        const double at = one_way ? -3.5 : (chain ? 0.5 : 0.0);  // anchor uc
                        const double t1 = 2.0 * a2 * X + bb * Y + cc * Z;
                        rec[3] = (float)(t0 - at * t1 + (chain ? (double)gt.off + (double)K : 0.0));
                        rec[4] = (float)(ty - at * (double)rec[1]);
                        rec[5] = (float)(tz - at * (double)rec[2]);
                        // C = 1: the weight I * 2^-off in units of kAccUnit, ~1 (see
                        // kAccUnit); the chains carry it in their factors
                        const float rho = C == 1 ? (I[0] * gt.fscale) * kInvAccUnit : 1.f;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float uc = 0.5f + (float)k;
                            // 2^-K applied exactly: the exp2 argument stays small
                            const float Gk = ldexpf(__builtin_amdgcn_exp2f(A2 * (uc * uc)), -(int)K);
                            rec[9 + k] = chain ? Gk * rho : fmaf(A2, uc * uc, gt.off);
                        }
#pragma unroll
                        for (int c = 0; c < C; ++c) rec[13 + c] = C == 1 ? rho : I[c] * gt.fscale;
                    } else {
                        // (cx, cy, cz, A2 | B, C, D, E | F, shift, half, - | I*2^shift)
                        rec[0] = cx; rec[1] = cy; rec[2] = cz; rec[3] = A2;
                        rec[4] = q1.x; rec[5] = q1.y; rec[6] = q1.z; rec[7] = q1.w;
                        rec[8] = F; rec[9] = gt.shift; rec[10] = gt.half; rec[11] = 0.f;
#pragma unroll
                        for (int c = 0; c < C; ++c)
                            rec[12 + c] = C == 1 ? (I[0] * gt.scale) * kInvAccUnit : I[c] * gt.scale;
                    }
#pragma unroll
                    for (int q = 0; q < kRecF4<C>; ++q)
                        s_rec[lane][q] = make_float4(rec[4 * q], rec[4 * q + 1], rec[4 * q + 2],
                                                     rec[4 * q + 3]);
                }
            }
            if (pair_live != nullptr) pair_live[idx] = live ? 1 : 0;
        }
        const uint64_t live_mask = __ballot(live);
        const uint64_t fast_mask = __ballot(fast);    // fast implies live
        const uint64_t chain_mask = __ballot(chain);  // chain implies fast
        uint64_t omask = __ballot(one_way);           // one_way implies chain
        uint64_t cmask = chain_mask & ~omask;
        uint64_t fmask = fast_mask & ~chain_mask;
        uint64_t smask = live_mask & ~fast_mask;
        __syncthreads();
        // One-way and centre-out chained Gaussians, then the other gate-free
        // ones, then the exact-gate ones of the batch: single-path loops keep the
        // accumulators in place (no copies per trip).
        while (omask) {
            const int j = __builtin_ctzll(omask);
            omask &= omask - 1;
            const float4 r0 = s_rec[j][0], r1 = s_rec[j][1], r2 = s_rec[j][2], r3 = s_rec[j][3];
            float iw[4];  // entries >= C are unused
            iw[0] = r3.y;
            if (C > 1) iw[1] = r3.z;
            if (C > 2) iw[2] = r3.w;
            if (C > 3) iw[3] = s_rec[j][kRecF4<C> - 1].x;
            const float T1 = fmaf(r0.y, py, fmaf(r0.z, pz, r0.x));
            const float E0 =  // E at uc = -3.5
                fmaf(r2.x, pz2, fmaf(r1.w, pyz, fmaf(r1.z, py2, fmaf(r1.y, pz, fmaf(r1.x, py, r0.w)))));
            const float G[4] = {r2.y, r2.z, r2.w, r3.x};  // 2^(A2 uc^2 - K), |uc| = 0.5 .. 3.5
            // two v_exp_f32 per row: 2^E at uc = -3.5 and the step 2^-T1 towards
            // +x; every product below 2^-126 is 0 (binary32 flush-to-zero mode),
            // which is the gate, as v_exp_f32's own flush is on the other paths
            const float step = __builtin_amdgcn_exp2f(-T1);
            float e = __builtin_amdgcn_exp2f(E0);
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u) {
                const float a = e * G[u < 4 ? 3 - u : u - 4];
                if (C == 1) {
                    acc[u][0] = add_nc(acc[u][0], a);  // a = I alpha / kAccUnit, gated
                } else {
#pragma unroll
                    for (int c = 0; c < C; ++c) acc[u][c] = fmaf(a, iw[c], acc[u][c]);
                }
                if (u + 1 < GSV_TILE) e *= step;
            }
        }
        while (cmask) {
            const int j = __builtin_ctzll(cmask);
            cmask &= cmask - 1;
            const float4 r0 = s_rec[j][0], r1 = s_rec[j][1], r2 = s_rec[j][2], r3 = s_rec[j][3];
            float iw[4];  // entries >= C are unused
            iw[0] = r3.y;
            if (C > 1) iw[1] = r3.z;
            if (C > 2) iw[2] = r3.w;
            if (C > 3) iw[3] = s_rec[j][kRecF4<C> - 1].x;
            const float T1 = fmaf(r0.y, py, fmaf(r0.z, pz, r0.x));
            const float E0 =  // E at uc = +0.5
                fmaf(r2.x, pz2, fmaf(r1.w, pyz, fmaf(r1.z, py2, fmaf(r1.y, pz, fmaf(r1.x, py, r0.w)))));
            const float G[4] = {r2.y, r2.z, r2.w, r3.x};  // 2^(A2 uc^2 - K), |uc| = 0.5 .. 3.5
            // three v_exp_f32 per row: 2^E at uc = +0.5 and the steps 2^-T1
            // (towards +x) and 2^T1 (towards -x); uc = -0.5 is the first step
            // left of it, so the chain spans 4 units of uc on the left
            const float step_r = __builtin_amdgcn_exp2f(-T1), step_l = __builtin_amdgcn_exp2f(T1);
            float er = __builtin_amdgcn_exp2f(E0);
            float el = er * step_l;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float ar = er * G[k], al = el * G[k];
                if (C == 1) {
                    acc[4 + k][0] = add_nc(acc[4 + k][0], ar);
                    acc[3 - k][0] = add_nc(acc[3 - k][0], al);
                } else {
#pragma unroll
                    for (int c = 0; c < C; ++c) {
                        acc[4 + k][c] = fmaf(ar, iw[c], acc[4 + k][c]);
                        acc[3 - k][c] = fmaf(al, iw[c], acc[3 - k][c]);
                    }
                }
                if (k < 3) {
                    er *= step_r;
                    el *= step_l;
                }
            }
        }
        while (fmask) {
            const int j = __builtin_ctzll(fmask);
            fmask &= fmask - 1;
            const float4 r0 = s_rec[j][0], r1 = s_rec[j][1], r2 = s_rec[j][2], r3 = s_rec[j][3];
            float iw[4];  // entries >= C are unused
            iw[0] = r3.y;
            if (C > 1) iw[1] = r3.z;
            if (C > 2) iw[2] = r3.w;
            if (C > 3) iw[3] = s_rec[j][kRecF4<C> - 1].x;
            const float T1 = fmaf(r0.y, py, fmaf(r0.z, pz, r0.x));
            const float T0 =
                fmaf(r2.x, pz2, fmaf(r1.w, pyz, fmaf(r1.z, py2, fmaf(r1.y, pz, fmaf(r1.x, py, r0.w)))));
            // s(u) = T0 - T1 uc + A2 uc^2 + off; voxels u and 7-u share uc^2
            const float V[4] = {T0 + r2.y, T0 + r2.z, T0 + r2.w, T0 + r3.x};
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u) {
                const float uc = (float)u - 3.5f;
                const int k = u < 4 ? 3 - u : u - 4;
                const float a = __builtin_amdgcn_exp2f(fmaf(-uc, T1, V[k]));
#pragma unroll
                for (int c = 0; c < C; ++c) acc[u][c] = fmaf(a, iw[c], acc[u][c]);
            }
        }
        while (smask) {
            const int j = __builtin_ctzll(smask);
            smask &= smask - 1;
            const float4 r0 = s_rec[j][0], r1 = s_rec[j][1], r2 = s_rec[j][2], r3 = s_rec[j][3];
            const float iw[4] = {r3.x, r3.y, r3.z, r3.w};
            const float dy = r0.y - py, dz = r0.z - pz;
            const float R1 = fmaf(r1.x, dy, r1.y * dz);
            const float R0 = fmaf(fmaf(r1.z, dy, r1.w * dz), dy, fmaf(r2.x * dz, dz, -r2.y));
            // along the row: s(u') = R0 + dx * (R1 + A2 * dx), dx = cx - u', in
            // the offsets themselves as the reference forms sigma (no expansion
            // about the row centre, whose terms would cancel for a large conic)
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u) {
                const float dx = r0.x - ((float)u - 3.5f);
                const float s = fmaf(dx, fmaf(r0.w, dx, R1), R0);
                const float a = (fabsf(s) <= r2.z) ? __builtin_amdgcn_exp2f(s) : 0.f;
#pragma unroll
                for (int c = 0; c < C; ++c) acc[u][c] = fmaf(a, iw[c], acc[u][c]);
            }
        }
        __syncthreads();
    }
    if (C == 1) {
#pragma unroll
        for (int u = 0; u < GSV_TILE; ++u) acc[u][0] *= kAccUnit;
    }
    const int y = tg.y0 + (lane & 7), z = tg.z0 + (lane >> 3);
    float lsum = 0.f;  // fused L1: sum of |volume - target| over the lane's row
    if (y < H && z < D) {
        const int64_t off = (((int64_t)z * H + y) * W + tg.x0) * C;
        float *o = vol + off;
        const int nx = min(GSV_TILE, W - tg.x0);
        constexpr int kRowF4 = 2 * C;  // float4s in a full row of 8 voxels
        if (nx == GSV_TILE && aligned_to(o, 16) &&
            (target == nullptr || (aligned_to(target + off, 16) && aligned_to(sgn + off, 8)))) {
            // whole row, vector accesses: 2C float4 stores, and for the fused
            // L1 2C float4 loads and C 8-byte stores of the sign bytes
            float v[GSV_TILE * C];
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u)
#pragma unroll
                for (int c = 0; c < C; ++c) v[u * C + c] = acc[u][c];
            float4 t4[kRowF4];
            if (target != nullptr) {
#pragma unroll
                for (int q = 0; q < kRowF4; ++q)
                    t4[q] = reinterpret_cast<const float4 *>(target + off)[q];
            }
#pragma unroll
            for (int q = 0; q < kRowF4; ++q)
                reinterpret_cast<float4 *>(o)[q] =
                    make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
            if (target != nullptr) {
                uint32_t words[kRowF4];
#pragma unroll
                for (int q = 0; q < kRowF4; ++q) {
                    const float tq[4] = {t4[q].x, t4[q].y, t4[q].z, t4[q].w};
                    uint32_t wd = 0;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float d = v[4 * q + b] - tq[b];
                        lsum += fabsf(d);
                        const int8_t sb = l1_sign(v[4 * q + b], tq[b]);
                        wd |= (uint32_t)(uint8_t)sb << (8 * b);
                    }
                    words[q] = wd;
                }
#pragma unroll
                for (int q = 0; q < C; ++q)
                    reinterpret_cast<uint2 *>(sgn + off)[q] = make_uint2(words[2 * q], words[2 * q + 1]);
            }
        } else {  // a partial edge row, or unaligned buffers: element by element
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u)
                if (u < nx)
#pragma unroll
                    for (int c = 0; c < C; ++c) o[u * C + c] = acc[u][c];
            if (target != nullptr) {
                const float *tt = target + off;
                int8_t *sg = sgn + off;
#pragma unroll
                for (int u = 0; u < GSV_TILE; ++u)
                    if (u < nx)
#pragma unroll
                        for (int c = 0; c < C; ++c) {
                            const float d = acc[u][c] - tt[u * C + c];
                            lsum += fabsf(d);
                            sg[u * C + c] = l1_sign(acc[u][c], tt[u * C + c]);
                        }
            }
        }
    }
    if (target != nullptr) {  // fixed-order wave sum, one partial per tile
#pragma unroll
        for (int o = kWave / 2; o >= 1; o >>= 1) lsum += __shfl_xor(lsum, o, kWave);
        if (lane == 0) tile_loss[tile] = lsum;
    }
    if (timeline && lane == 0) wave_rec[3 * (int64_t)blockIdx.x + 1] = wall_clock64();
}

// loss = (sum over tiles of the partials) / numel, summed in a fixed order in
// binary64 by one workgroup: float4 loads (when the partials are 16-byte
// aligned) into four running sums per thread keep many loads in flight.
constexpr int kFinishThreads = 1024;

__global__ __launch_bounds__(kFinishThreads) void k_loss_finish(const float *__restrict__ tile_loss,
                                                                int64_t T, double numel,
                                                                float *__restrict__ loss) {
    __shared__ double s_w[kFinishThreads / kWave];
    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
    const int64_t T4 = aligned_to(tile_loss, 16) ? T / 4 : 0;
    const float4 *t4 = reinterpret_cast<const float4 *>(tile_loss);
#pragma unroll 16
    for (int64_t i = threadIdx.x; i < T4; i += kFinishThreads) {
        const float4 v = t4[i];
        a0 += (double)v.x;
        a1 += (double)v.y;
        a2 += (double)v.z;
        a3 += (double)v.w;
    }
    for (int64_t i = 4 * T4 + threadIdx.x; i < T; i += kFinishThreads) a0 += (double)tile_loss[i];
    double acc = (a0 + a1) + (a2 + a3);
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) s_w[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < kFinishThreads / kWave; ++w) t += s_w[w];
        *loss = (float)(t / numel);
    }
}

// --------------------------------------------------------------- backward --

// pair_tiles[p] = tile of sorted pair p: one wave per tile writes its range.
// Only needed when the caller has not kept the binning's sorted keys.
__global__ __launch_bounds__(kWave) void k_pair_tiles(const int2 *__restrict__ bins, int n_isect,
                                                      int *__restrict__ pair_tiles) {
    const int t = blockIdx.x;
    const int2 r = bins[t];
    const int e = min(r.y, n_isect);
    for (int q = max(r.x, 0) + (int)threadIdx.x; q < e; q += kWave) pair_tiles[q] = t;
}

template <int C>
struct Moments {
    float S0, Sx, Sy, Sz, Sxx, Sxy, Sxz, Syy, Syz, Szz;
    float dI[C];
};

// The quadratic form of a gate-free pair in the LDL^T coordinates of its conic,
// about the tile centre.  With delta = mu - p = m - p' (m the Gaussian's
// centre relative to the tile centre, p' = local voxel index - 3.5 per axis),
// Q = L D L^T (L unit lower triangular) and k = log2(e) / 2,
//   sigma2 = -k delta^T Q delta = -(tau^2 + eta^2 + zeta^2),
//   tau  = sqrt(k D1) (delta_x + l21 delta_y + l31 delta_z) = tc - al p'x - be p'y - ga p'z,
//   eta  = sqrt(k D2) (delta_y + l32 delta_z)               = ec - be2 p'y - ga2 p'z,
//   zeta = sqrt(k D3) delta_z                               = zc - ga3 p'z.
// sigma2 is then a sum of squares of quantities that are small wherever a
// voxel weighs (|tau|, |eta|, |zeta| <= sqrt(-t2) inside the gate), so its
// binary32 rounding stays near that of sigma2 itself.  The expanded form
// A2 dx^2 + dx (Bn dy + Cn dz) + ... sums terms of up to |Q| |delta|^2 that
// cancel for an elongated, rotated Gaussian (terms of ~1e3 for a sum of ~10
// on a 0.5 x 6 voxel Gaussian 15 voxels from its centre), and their rounding
// is shared by whole rows (R0, R1) or by the whole Gaussian (the scaled
// coefficients), so it does not average out of the gradient sums: ~30x the
// reference's error on its worst dconics elements.  The tile-centre terms tc,
// ec, zc are formed in binary64 from the binary64 factor; the per-row and
// per-voxel coefficients multiply |p'| <= 3.5 only, so their binary32
// rounding costs little.
struct RowForm {
    float al, be, ga, be2, ga2, ga3;  // coefficients of p'
    float tc, ec, zc;                 // tau, eta, zeta at the tile centre
};

// The part of the row form that depends on the conic alone: the LDL^T factor
// (binary64 unit-triangle entries, binary32 square roots of the k-scaled
// pivots) and the binary32 coefficients of p'.
struct RowFactor {
    double l21, l31, l32;
    float al, b2, g3;   // sqrt(k D1), sqrt(k D2), sqrt(k D3)
    float be, ga, ga2;  // al l21, al l31, b2 l32
    float r_ell;        // w^T Q^-1 w, w = 2k (0, b, c): the slope's spread over the gate
};

// The LDL^T factor of a conic (binary64).  False (the Gaussian's pairs then
// take the exact path) unless the binary64 pivots are positive and each
// k * pivot lies in [2^-100, 2^100], where its binary32 square root is a
// normal number.  Zero coefficients otherwise.
__device__ __forceinline__ bool row_factor(float ca, float cb, float cc, float cd, float ce,
                                           float cf, RowFactor &F) {
    F.l21 = F.l31 = F.l32 = 0.0;
    F.al = F.b2 = F.g3 = F.be = F.ga = F.ga2 = F.r_ell = 0.f;
    constexpr double k = 0.72134752044448170368;  // log2(e) / 2
    const double a = ca, b = cb, c = cc, d = cd, e = ce, ff = cf;
    const double ia = 1.0 / a;
    const double l21 = b * ia, l31 = c * ia;
    const double d2 = fma(-b, l21, d), e2 = fma(-c, l21, e), f2 = fma(-c, l31, ff);
    const double l32 = e2 / d2;
    const double d3 = fma(-e2, l32, f2);
    const double p1 = k * a, p2 = k * d2, p3 = k * d3;
    constexpr double lo = 0x1p-100, hi = 0x1p100;
    if (!(p1 >= lo && p1 <= hi && p2 >= lo && p2 <= hi && p3 >= lo && p3 <= hi)) return false;
    const float al = __builtin_amdgcn_sqrtf((float)p1);
    const float b2 = __builtin_amdgcn_sqrtf((float)p2);
    F.l21 = l21; F.l31 = l31; F.l32 = l32;
    F.al = al;
    F.b2 = b2;
    F.g3 = __builtin_amdgcn_sqrtf((float)p3);
    F.be = (float)(al * l21);
    F.ga = (float)(al * l31);
    F.ga2 = (float)(b2 * l32);
    // y = L^-1 w, w = 2k (0, b, c): w^T Q^-1 w = y2^2 / D2 + y3^2 / D3
    const double y2 = 2.0 * k * b, y3 = fma(-l32, y2, 2.0 * k * c);
    F.r_ell = (float)(y2 * y2 / d2 + y3 * y3 / d3);
    return true;
}

// The row form of the pair whose Gaussian lies at (mx, my, mz) from the tile
// centre, from its factor's binary32 square roots al, b2, g3 and the binary64
// products be = al l21, ga = al l31, ga2 = b2 l32: the tile-centre terms in
// binary64 (al mx and b2 my are exact there), the coefficients their binary32
// roundings.
__device__ __forceinline__ void row_centre(float al, float b2, float g3, double be, double ga,
                                           double ga2, float mx, float my, float mz, RowForm &f) {
    f.al = al;
    f.be = (float)be;
    f.ga = (float)ga;
    f.be2 = b2;
    f.ga2 = (float)ga2;
    f.ga3 = g3;
    f.tc = (float)fma(ga, (double)mz, fma(be, (double)my, (double)al * (double)mx));
    f.ec = (float)fma(ga2, (double)mz, (double)b2 * (double)my);
    f.zc = g3 * mz;
}

// Adds to M the moments of h = a * G about the Gaussian's centre for one lane's pair:
// S[..] = sum h * delta^k, delta = mu - p, G = sum_c I_c g_c (g_c alone for
// C == 1; I folds into the final scale).  Per voxel: h, h*dx by an FMA against
// the lane's hoisted dx_u, and h into its column's sum (for Sxx); rows fold in
// dy, planes in dz.
// Taking moments about the Gaussian (not the tile) keeps every sum
// well-conditioned: h is large only where |delta| is small.
// The exponent a = 2^(sigma2 + ...) per mode:
//   kRowsForm (gate-free): sigma2 = -(t^2 + c_r) from the row form (RowForm),
//              t = tau = u_r - x_u with u_r = tau + al p'x per row and
//              x_u = al p'_u per lane, c_r = eta^2 + zeta^2 per row;
//              a = exp2(sigma2) * 2^off, zero below the threshold by the flush
//              of the product (off = the gate-free offset, one v_exp_f32 per
//              lane for 2^off).  The offset stays out of the exponent: an
//              argument near -100 rounds to ~8e-6 in binary32, ~3e-6 relative
//              in a;
//   kRowsChain (gate-free too): a row's a from three v_exp_f32 instead of
//              eight, as products, which the binary32 flush-to-zero mode gates
//              like v_exp_f32: a_u = 2^E_u * G_u with the lane's column factors
//              G_u = 2^(-x_u^2 - K) and E_u = sigma2_u + off + x_u^2 + K
//              = (off + K - c_r - u_r^2) + 2 u_r x_u, linear in x_u: 2^E at
//              u = 0 and u = 4, each stepped three times by 2^(2 al u_r).
//              chain_shift picks K, which keeps every factor finite and every
//              product of a chain up to a passing voxel above 2^-126.  Its
//              rounding: the step's exponent (|2 al u_r| up to ~40, rounded once
//              per row) and each anchor's (up to 3 columns from the voxels it
//              serves) enter up to 4 values at once, where the form path
//              rounds only per-voxel quantities near sigma2's own size; at cfg3
//              and cfg5 the chained rows leave ~1.5-3x as many gradient
//              elements as the form path outside rel 1e-4 / abs 1e-6 of the
//              binary64 value for an N(0,1) vol_grad, and run the backward
//              ~20 % faster (GSV_BWD_CHAIN=0 selects the form path);
//   kRowsExact: a = exp2(s) if |s| <= bound, s = sigma2 - shift, with sigma2 =
//              R0 + dx (R1 + A2 dx) from the scaled conic (R1 = Bn dy + Cn dz,
//              R0 = Dn dy^2 + En dy dz + Fn dz^2 per row): any conic, including
//              indefinite and non-finite ones, as the reference evaluates it.
constexpr int kRowsExact = 0, kRowsForm = 1, kRowsChain = 2;

template <int C, int kMode>
__device__ __forceinline__ void pair_moments(const float4 *s_rows, float mxl, float myl, float mzl,
                                             const RowForm &f, float A2, float Bn, float Cn,
                                             float Dn, float En, float Fn, float shift, float bound,
                                             float K, const float (&Gt)[GSV_TILE],
                                             const float (&I)[C], Moments<C> &M) {
    constexpr bool kForm = kMode != kRowsExact, kChain = kMode == kRowsChain;
    // Sxx is only needed whole: the loop sums h per voxel column (col[u], a
    // two-operand add per voxel) and Sxx = sum_u dx_u^2 col[u] is formed once at
    // the end, instead of an FMA chain against dx_u^2 in every row
    float dxu[GSV_TILE], col[GSV_TILE], xu[GSV_TILE];
#pragma unroll
    for (int u = 0; u < GSV_TILE; ++u) {
        dxu[u] = mxl - ((float)u - 3.5f);
        col[u] = 0.f;
        xu[u] = f.al * ((float)u - 3.5f);  // kForm: x_u = al p'_u
    }
    // kRowsForm: 2^off, a normal number on live lanes (off in [-126, -66]) and 0
    // at the dead offset, where the form is 0 (zero coefficients) and a = 1 * 0
    const float Fb = kMode == kRowsForm ? __builtin_amdgcn_exp2f(bound) : 0.f;
    // kRowsChain: G_u = 2^(-x_u^2 - K), Gt[u] = 2^(-x_u^2) being the
    // Gaussian's column factor (column_factors); 2^-K is applied exactly.
    float G[GSV_TILE];
    if (kChain) {
#pragma unroll
        for (int u = 0; u < GSV_TILE; ++u) G[u] = ldexpf(Gt[u], -(int)K);
    }
    // the per-plane constant: the chain's offset and K (its E), the exact
    // path's shift
    const float c0 = kChain ? bound + K : (kForm ? 0.f : -shift);
    for (int lz = 0; lz < GSV_TILE; ++lz) {
        const float pz = (float)lz - 3.5f;
        const float dz = mzl - pz;
        // kForm: zeta, then -zeta^2 + c0, and the plane's parts of tau and eta
        const float zt = kForm ? fmaf(-f.ga3, pz, f.zc) : 0.f;
        const float zz = kForm ? fmaf(-zt, zt, c0) : 0.f;
        const float tz = kForm ? fmaf(-f.ga, pz, f.tc) : 0.f;
        const float ez = kForm ? fmaf(-f.ga2, pz, f.ec) : 0.f;
        // kRowsExact: the plane's parts of R1 and R0
        const float Cdz = kForm ? 0.f : Cn * dz, Edz = kForm ? 0.f : En * dz;
        const float R0z = kForm ? 0.f : fmaf(Fn * dz, dz, c0);
        float Q0 = 0.f, Qx = 0.f, Qy = 0.f, Qxy = 0.f, Qyy = 0.f;
#pragma unroll
        for (int ly = 0; ly < GSV_TILE; ++ly) {
            const int row = lz * GSV_TILE + ly;
            float gv[GSV_TILE * C];
#pragma unroll
            for (int q = 0; q < 2 * C; ++q) {
                const float4 t4 = s_rows[row * 2 * C + q];
                gv[4 * q] = t4.x; gv[4 * q + 1] = t4.y; gv[4 * q + 2] = t4.z; gv[4 * q + 3] = t4.w;
            }
            const float py = (float)ly - 3.5f;
            const float dy = myl - py;
            float ur = 0.f, cr = 0.f, R1 = 0.f, R0 = 0.f;
            if (kForm) {
                ur = fmaf(-f.be, py, tz);              // u_r = tau + al p'x
                const float et = fmaf(-f.be2, py, ez);  // eta
                cr = fmaf(-et, et, zz);                 // -(eta^2 + zeta^2) (+ off + K)
            } else {
                R1 = fmaf(Bn, dy, Cdz);
                R0 = fmaf(fmaf(Dn, dy, Edz), dy, R0z);
            }
            float sv[GSV_TILE];  // kRowsChain: the row's a
            if (kChain) {
                // E_u = q + 2 u_r x_u (2 x_u and 2 al are exact doublings)
                const float q = fmaf(-ur, ur, cr);
                const float step = __builtin_amdgcn_exp2f(ur * (2.0f * f.al));      // 2^(2 al u_r)
                float e1 = __builtin_amdgcn_exp2f(fmaf(ur, 2.0f * xu[0], q));  // u = 0
                float e2 = __builtin_amdgcn_exp2f(fmaf(ur, 2.0f * xu[4], q));  // u = 4
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    sv[k] = e1 * G[k];
                    sv[4 + k] = e2 * G[4 + k];
                    if (k < 3) {
                        e1 *= step;
                        e2 *= step;
                    }
                }
            }
            float W1 = 0.f, h[GSV_TILE];
            // C > 1: the row's sums of a * g_c, added to the pair's totals once
            // per row (64 additions of row sums, not 512 running ones)
            float rI[C];
#pragma unroll
            for (int c = 0; c < C; ++c) rI[c] = 0.f;
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u) {
                float a;
                if (kChain) {
                    a = sv[u];
                } else if (kForm) {
                    const float t = ur - xu[u];
                    a = __builtin_amdgcn_exp2f(fmaf(-t, t, cr)) * Fb;  // flushed below 2^-126: the gate
                } else {
                    const float s = fmaf(dxu[u], fmaf(dxu[u], A2, R1), R0);
                    a = (fabsf(s) <= bound) ? __builtin_amdgcn_exp2f(s) : 0.f;
                }
                if (C == 1) {
                    h[u] = a * gv[u];
                } else {
                    float Gs = 0.f;
#pragma unroll
                    for (int c = 0; c < C; ++c) {
                        Gs = fmaf(I[c], gv[u * C + c], Gs);
                        rI[c] = fmaf(a, gv[u * C + c], rI[c]);
                    }
                    h[u] = a * Gs;
                }
                W1 = fmaf(h[u], dxu[u], W1);
                col[u] = add_nc(col[u], h[u]);
            }
            if (C > 1) {
#pragma unroll
                for (int c = 0; c < C; ++c) M.dI[c] = add_nc(M.dI[c], rI[c]);
            }
            // the row sum of the h already formed: 7 two-operand adds, which
            // issue faster than the 8 three-operand FMAs a contracted a*g sum takes
            const float W0 = add_nc(add_nc(add_nc(h[0], h[1]), add_nc(h[2], h[3])),
                                    add_nc(add_nc(h[4], h[5]), add_nc(h[6], h[7])));
            Q0 += W0;
            Qx += W1;
            Qy = fmaf(W0, dy, Qy);
            Qxy = fmaf(W1, dy, Qxy);
            Qyy = fmaf(W0, dy * dy, Qyy);
        }
        M.S0 += Q0;
        M.Sx += Qx;
        M.Sy += Qy;
        M.Sxy += Qxy;
        M.Syy += Qyy;
        M.Sz = fmaf(Q0, dz, M.Sz);
        M.Sxz = fmaf(Qx, dz, M.Sxz);
        M.Syz = fmaf(Qy, dz, M.Syz);
        M.Szz = fmaf(Q0, dz * dz, M.Szz);
    }
    float sxx = 0.f;
#pragma unroll
    for (int u = 0; u < GSV_TILE; ++u) sxx = fmaf(dxu[u] * dxu[u], col[u], sxx);
    M.Sxx += sxx;
}

// vol_grad of a tile is staged scaled by a power of two so that its largest
// magnitude lies in [2^89, 2^90): with the gate-free a >= 2^-126, every
// h = a * G is then a normal number whatever the loss scale.  The epilogue
// divides the factor out.
constexpr int kGradScaleExp = 90;

// Tiles staged at once by a backward wave: the LDS of K tiles (2 KB * C each)
// must leave room for several waves per CU.  Sparse scenes stage more: their
// 64-pair waves span several tiles, and every tile beyond K costs the wave
// another 64-row pass in k_vox_bwd_rest, far more than the occupancy the
// larger LDS share takes.  By the mean pairs per tile (measured on 512^3
// scenes: 17 per tile, C = 1: K = 8 684 us, 6 920 us, 3 2254 us; 41 per tile:
// K = 6 1252 us, 8 1358 us, 3 1600 us; 81 and 108 per tile: K = 3 best;
// 17 per tile at C = 4: K = 6 2805 us, 4 4060 us; at C = 2: 1415, 2550 us):
template <int C>
constexpr int kStageTiles = C == 1 ? 3 : 2;          // >= kSparsePairs per tile
template <int C>
constexpr int kStageTilesSparse = C == 1 ? 6 : 4;    // < kSparsePairs
template <int C>
constexpr int kStageTilesVerySparse = C == 1 ? 8 : 6;  // < kVerySparsePairs
constexpr int64_t kSparsePairs = 64;
constexpr int64_t kVerySparsePairs = 24;

// Whether the backward may take chained rows: on, unless GSV_BWD_CHAIN=0 is
// set when the process first asks, or gsv_set_backward_chains(0) was called.
// Read once per process, then kept here.
std::atomic<int> g_bwd_chains{-1};

bool bwd_chains_enabled() {
    int v = g_bwd_chains.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *env = getenv("GSV_BWD_CHAIN");
        int unset = -1;
        g_bwd_chains.compare_exchange_strong(unset, (env && strcmp(env, "0") == 0) ? 0 : 1);
        v = g_bwd_chains.load(std::memory_order_relaxed);
    }
    return v != 0;
}

struct BwdArgs {
    int D, H, W, Tx, Ty, n, n_isect;
    FastDiv fx, fy;  // division by Tx and by Ty
    // Chained rows allowed (bwd_chains_enabled()).  A group takes them
    // when every one of its pairs qualifies, so a pair's rounding can depend on
    // the pairs it shares a wave with (as for exact-gate pairs, which take the
    // whole group to the exact path); without them it never does.
    int chain;
    int64_t T;
    const int *ids, *pair_tiles;
    const float4 *pos_radii;
    const float2 *conics;
    const float *intens, *vol_grad;
    const int8_t *l1_sgn;
    const float *l1_grad;
    float l1_numel;
    float *dpos, *dconic, *dint;
    const int *tile_min, *tile_max, *cum;
    // The per-Gaussian records k_bwd_prep wrote (kBwdRecF4 float4 per Gaussian)
    const float4 *rec;
    float *partial;
    const int64_t *d_count;  // live pair count on the device (n_isect is then the capacity)
    // Optional work list: order[0 .. *d_work) holds the sorted positions of the
    // pairs the forward's tile culling kept, ascending, and order[n_isect - 1],
    // order[n_isect - 2], ... the culled ones, whose zero partials k_vox_bwd
    // writes.  Without it the work is every pair.
    const int *order;
    const int64_t *d_work;
    int n_work;  // work items, set by each kernel from the counts
    // One byte per wave of work items, written by k_vox_bwd for every wave:
    // 1 when the wave's pairs span more tiles than it stages (k_vox_bwd_rest
    // processes the others).
    uint8_t *rest_flag;
};

// The live pair count: *d_count clamped to [0, cap], or cap without one.
__device__ __forceinline__ int live_pairs(int cap, const int64_t *d_count) {
    if (!d_count) return cap;
    const int64_t v = *d_count;
    return v < 0 ? 0 : (v < cap ? (int)v : cap);
}

// Sets a.n_isect to the live pair count and a.n_work to the work items.
__device__ __forceinline__ void bwd_counts(BwdArgs &a) {
    a.n_isect = live_pairs(a.n_isect, a.d_count);
    a.n_work = a.order ? live_pairs(a.n_isect, a.d_work) : a.n_isect;
}

// Sorted position of work item q (q < a.n_work).
__device__ __forceinline__ int bwd_pair(const BwdArgs &a, int64_t q) {
    return a.order ? a.order[q] : (int)q;
}

// One backward wave's view: lane = one of 64 consecutive work items (pairs of
// the sorted list, or of the work list of kept pairs); `slot` numbers the runs
// of equal tiles.
template <int C>
struct BwdLane {
    int tile, slot, g, p;
    bool valid, live, fast;
    float mxl, myl, mzl;
    float I[C];
    float off, fscale;  // the gate-free path's offset and its 2^-off
    TileGeom tg;
    RowForm rf;  // gate-free pairs: the row form about the tile centre
    float kch;   // gate-free pairs: chain_shift's K, or -1
    int slot_e;  // deterministic mode: the pair's emission slot (< 2^31), or -1
    const float4 *rp;  // the Gaussian's record (valid lanes with a Gaussian in range)
};

// ---------------------------------------------- per-Gaussian backward record --
//
// Everything a backward pair reads of its Gaussian, and the parts of its
// set-up that do not depend on the tile, in one 128-byte record (one cache
// line) per Gaussian: the centre, the gate, the LDL^T factor of the conic,
// the tile-independent terms of the chain's shift bound, the column factors
// 2^(-x_u^2), the first channel's intensity and the emission box.
// k_bwd_prep forms them once per Gaussian (one lane each) instead of once per
// (tile, Gaussian) pair (~16 pairs per Gaussian at 256^3 / 200k: the factor's
// four binary64 divisions, the gate's log2, the column factors' exp2), and a
// pair reads one line where its position, conic, intensity, box and cum
// gathers touched six to nine.  The conic itself is not needed: the
// deterministic mode applies it per Gaussian in k_pair_reduce.  float4 fields:
//   0  px, py, pz, flags          1  off, s_ell, m_reach, al
//   2  b2, g3, I0, t2             3  al l21, al l31 (binary64)
//   4  b2 l32 (binary64), ebase   5  extent x, extent y, cum[g-1], cum[g]
//   6  Gt[0..3]                   7  Gt[4..7]
// ebase (int64) = cum[g-1] - (min.z * ny + min.y) * nx - min.x, so that a
// pair's emission slot is ebase + (tz * ny + ty) * nx + tx; the ints of
// field 5 are nx, ny and the Gaussian's slot range.  The chain terms (see
// chain_shift): m_reach = 2 al^2 (3.5 + sqrt(k2 / a)), s_ell = sqrt(k2 r_ell),
// k2 = -2 ln2 t2; the pair forms k_max = floor(120 - 12.25 al^2), rint(-off)
// and 2^-off itself.  Bits of flags: kRecLive (the gate can pass),
// kRecBounded (a finite positive mean), kRecFast (gate-free with a valid row
// factor).  The factor, chain and column fields are zero unless kRecFast; the
// box fields are zero in the atomic mode, which has none.
constexpr int kBwdRecF4 = 8;
constexpr unsigned kRecLive = 1u, kRecFast = 2u, kRecBounded = 4u;
constexpr int kPrepThreads = 256;
constexpr int kPrepStride = kBwdRecF4 + 1;  // LDS float4 per staged record: +1 spreads the banks

// Column factors of the chained rows: Gt[u] = 2^(-x_u^2) at the positions the
// chain implies, x_u = x_a + (u - a) al from its anchor a (0 or 4; x_0 and x_4
// as the anchors' exponents take them: fl(al * -3.5) and al / 2 exactly) and
// the step's exact multiples of al: x_u^2 in binary64, its binary32 rounding
// residual applied as the factor 1 + lo ln 2, so each factor is within ~1e-7
// of its value.  (Factors from the separately rounded al p'_u instead differ
// from the chain's exponents by 2 u_r (x_u - x_a - (u - a) al), the same in
// every row and tile of the Gaussian, which does not average out of its sums:
// at cfg5 1.3x as many dpos and dintensities elements outside rel 1e-4 /
// abs 1e-6 for an N(0,1) vol_grad.)
__device__ __forceinline__ void column_factors(float al, float (&Gt)[GSV_TILE]) {
    const float x0 = al * (0.0f - 3.5f), x4 = al * (4.0f - 3.5f);
#pragma unroll
    for (int u = 0; u < GSV_TILE; ++u) {
        const double xe = (double)(u < 4 ? x0 : x4) + (double)al * (u < 4 ? u : u - 4);
        const double d = -xe * xe;
        const float hi = (float)d;
        const float lo = (float)(d - (double)hi);
        Gt[u] = __builtin_amdgcn_exp2f(hi) * fmaf(lo, kLn2, 1.0f);
    }
}

// The record pass's inputs and output.  tile_min, tile_max and cum are NULL
// in the atomic mode.
struct PrepArgs {
    int n;
    const float4 *pos_radii;
    const float2 *conics;
    const float *intens;
    const int *tile_min, *tile_max, *cum;
    float4 *rec;
};

// Block `blk` of the record pass: one lane per Gaussian, its record (layout
// above) staged in LDS (s_rec: kPrepThreads * kPrepStride float4) so that the
// block writes its 256 records as one coalesced run (scattered 16-byte stores
// at the record stride take twice as long).
template <int C>
__device__ __forceinline__ void bwd_prep_block(int blk, const PrepArgs &P, float4 *s_rec) {
    const int n = P.n;
    const float4 *__restrict__ pos_radii = P.pos_radii;
    const float2 *__restrict__ conics = P.conics;
    const float *__restrict__ intens = P.intens;
    const int *__restrict__ tile_min = P.tile_min, *__restrict__ tile_max = P.tile_max;
    const int *__restrict__ cum = P.cum;
    float4 *__restrict__ rec = P.rec;
    const int t = (int)threadIdx.x, g0 = blk * kPrepThreads, g = g0 + t;
    if (g < n) {
        const float4 pr = pos_radii[g];
        const float2 c01 = conics[3 * g], c23 = conics[3 * g + 1], c45 = conics[3 * g + 2];
        float I0 = 0.f, mean = 0.f, max_abs = 0.f;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const float v = intens[(size_t)g * C + c];
            if (c == 0) I0 = v;
            mean += v;
            max_abs = fmaxf(max_abs, fabsf(v));
        }
        mean /= (float)C;
        const Gate gt = make_gate(mean);
        unsigned flags = (gt.live ? kRecLive : 0u) | (gt.bounded ? kRecBounded : 0u);
        RowFactor F{};
        bool fast = gt.live && gate_free_ok(gt, max_abs, pr.x, pr.y, pr.z, c01.x, c01.y, c23.x,
                                            c23.y, c45.x, c45.y);
        if (fast) fast = row_factor(c01.x, c01.y, c23.x, c23.y, c45.x, c45.y, F);
        float s_ell = 0.f, m_reach = 0.f;
        double be_d = 0.0, ga_d = 0.0, ga2_d = 0.0;
        float Gt[GSV_TILE];
#pragma unroll
        for (int u = 0; u < GSV_TILE; ++u) Gt[u] = 0.f;
        if (fast) {
            flags |= kRecFast;
            const float a2 = F.al * F.al;
            const float k2 = -2.0f * kLn2 * gt.t2;
            m_reach = 2.0f * a2 *
                      (3.5f + __builtin_amdgcn_sqrtf(fmaxf(k2 * __builtin_amdgcn_rcpf(c01.x), 0.f)));
            s_ell = __builtin_amdgcn_sqrtf(fmaxf(k2 * F.r_ell, 0.f));
            be_d = F.al * F.l21;
            ga_d = F.al * F.l31;
            ga2_d = F.b2 * F.l32;
            column_factors(F.al, Gt);
        }
        int nx = 0, ny = 0, base = 0, end = 0;
        int64_t ebase = 0;
        if (cum != nullptr) {
            const int mnx = tile_min[3 * g], mny = tile_min[3 * g + 1], mnz = tile_min[3 * g + 2];
            nx = tile_max[3 * g] - mnx;
            ny = tile_max[3 * g + 1] - mny;
            base = g == 0 ? 0 : cum[g - 1];
            end = cum[g];
            ebase = (int64_t)base - ((int64_t)mnz * ny + mny) * nx - mnx;
        }
        const auto bits = [](int v) { return __int_as_float(v); };
        const auto dlo = [](double v) {
            return __int_as_float((int)(uint32_t)__double_as_longlong(v));
        };
        const auto dhi = [](double v) {
            return __int_as_float((int)(uint32_t)((uint64_t)__double_as_longlong(v) >> 32));
        };
        const double eb = __longlong_as_double((long long)ebase);  // the int64's bits
        float4 *r = s_rec + t * kPrepStride;
        r[0] = make_float4(pr.x, pr.y, pr.z, bits((int)flags));
        r[1] = make_float4(gt.off, s_ell, m_reach, F.al);
        r[2] = make_float4(F.b2, F.g3, I0, gt.t2);
        r[3] = make_float4(dlo(be_d), dhi(be_d), dlo(ga_d), dhi(ga_d));
        r[4] = make_float4(dlo(ga2_d), dhi(ga2_d), dlo(eb), dhi(eb));
        r[5] = make_float4(bits(nx), bits(ny), bits(base), bits(end));
        r[6] = make_float4(Gt[0], Gt[1], Gt[2], Gt[3]);
        r[7] = make_float4(Gt[4], Gt[5], Gt[6], Gt[7]);
    }
    __syncthreads();
    const int cnt = min(kPrepThreads, n - g0) * kBwdRecF4;  // g0 < n: the grid covers n exactly
    float4 *dst = rec + (size_t)g0 * kBwdRecF4;
    for (int i = t; i < cnt; i += kPrepThreads)
        dst[i] = s_rec[(i / kBwdRecF4) * kPrepStride + (i % kBwdRecF4)];
}

// The record pass alone (the backward without a work list).
template <int C>
__global__ __launch_bounds__(kPrepThreads) void k_bwd_prep(PrepArgs P) {
    __shared__ float4 s_rec[kPrepThreads * kPrepStride];
    bwd_prep_block<C>((int)blockIdx.x, P, s_rec);
}

__device__ __forceinline__ double rec_double(float lo, float hi) {
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)__float_as_int(hi) << 32) |
                                            (uint64_t)(uint32_t)__float_as_int(lo)));
}

// Emission slot of the pair (tile, g): e = cum[g-1] + ((tz-min.z)*ny +
// (ty-min.y))*nx + (tx-min.x), the order the pairs were duplicated in
// (gaussian-major, tiles z->y->x), so each Gaussian's partials are contiguous
// for the reduction pass.  -1 when g or the tile is out of range or the slot
// lies outside [cum[g-1], cum[g]) or past the pair count.
__device__ __forceinline__ int64_t emission_slot_at(int g, int tx, int ty, int tz, int n,
                                                    const int *tile_min, const int *tile_max,
                                                    const int *cum, int n_isect) {
    if ((unsigned)g >= (unsigned)n) return -1;
    const int mnx = tile_min[3 * g], mny = tile_min[3 * g + 1], mnz = tile_min[3 * g + 2];
    const int nxb = tile_max[3 * g] - mnx, nyb = tile_max[3 * g + 1] - mny;
    const int64_t base = g == 0 ? 0 : cum[g - 1];
    const int64_t e = base + ((int64_t)(tz - mnz) * nyb + (ty - mny)) * nxb + (tx - mnx);
    return (e >= base && e < (int64_t)cum[g] && e < n_isect) ? e : -1;
}

__device__ __forceinline__ int64_t emission_slot(int g, int tile, const BwdArgs &a) {
    if ((unsigned)g >= (unsigned)a.n || tile < 0) return -1;
    const unsigned qt = fastdiv((unsigned)tile, a.fx);
    const int tx = (int)((unsigned)tile - qt * (unsigned)a.Tx);
    const unsigned tz = fastdiv(qt, a.fy);
    const int ty = (int)(qt - tz * (unsigned)a.Ty);
    return emission_slot_at(g, tx, ty, (int)tz, a.n, a.tile_min, a.tile_max, a.cum, a.n_isect);
}

// The forward's tile culling (pair_live: one byte per sorted pair) as the
// backward's work list.  order[0 .. kept) = the sorted positions of the pairs
// the forward kept, ascending; order[np-1], order[np-2], ... = the culled
// ones (np = the pair count).  Two passes over 4096 flags per block: counts,
// then positions (each block adds its predecessors' counts itself up to 2048
// blocks; beyond that one workgroup scans the counts in between).
constexpr int kKeepThreads = 256;
constexpr int kKeepItems = 16;
constexpr int kKeepTile = kKeepThreads * kKeepItems;
static_assert(kKeepThreads == scan_detail::kThreads, "block scan of gsv_scan.h");

// Flags [i0, i0 + 16) as a bit mask (bit k: pair i0 + k kept); *valid = how
// many of them lie below the pair count np.
__device__ __forceinline__ unsigned keep_mask(const uint8_t *flags, int64_t i0, int np,
                                              int *valid) {
    const int64_t v = min<int64_t>(kKeepItems, (int64_t)np - i0);
    *valid = v > 0 ? (int)v : 0;
    unsigned m = 0;
    if (v >= kKeepItems) {
        const uint4 w = *reinterpret_cast<const uint4 *>(flags + i0);
        const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                if ((ws[q] >> (8 * b)) & 0xffu) m |= 1u << (4 * q + b);
    } else {
        for (int k = 0; k < *valid; ++k)
            if (flags[i0 + k]) m |= 1u << k;
    }
    return m;
}

// Blocks [0, nprep): the record pass (bwd_prep_block); blocks nprep + b: the
// kept count of flags [4096 b, 4096 (b + 1)) into part[b].  The two are
// independent, so one launch runs them side by side: the counts take ~5 us
// as a launch of their own, and run under the record pass here.
template <int C>
__global__ __launch_bounds__(kKeepThreads) void k_keep_count(const uint8_t *__restrict__ flags,
                                                             int cap,
                                                             const int64_t *__restrict__ d_count,
                                                             int32_t *__restrict__ part,
                                                             int nprep, PrepArgs P) {
    static_assert(kKeepThreads == kPrepThreads, "one block size for both");
    __shared__ float4 s_rec[kPrepThreads * kPrepStride];
    __shared__ int lds_waves[kKeepThreads / kWave];
    if ((int)blockIdx.x < nprep) {  // uniform per block
        bwd_prep_block<C>((int)blockIdx.x, P, s_rec);
        return;
    }
    const int blk = (int)blockIdx.x - nprep;
    const int np = live_pairs(cap, d_count);
    const int64_t i0 = (int64_t)blk * kKeepTile + (int64_t)threadIdx.x * kKeepItems;
    int valid;
    const int c = __popc(keep_mask(flags, i0, np, &valid));
    int total;
    (void)scan_detail::block_exclusive(c, lds_waves, &total);
    if (threadIdx.x == 0) part[blk] = total;
}

// direct: part holds raw block counts (nb <= 2048); otherwise part holds their
// exclusive prefix and *d_kept the total already.  The block's kept positions
// (ascending) and culled ones (descending) are staged in LDS and stored as
// two contiguous runs.
__global__ __launch_bounds__(kKeepThreads) void k_keep_order(
    const uint8_t *__restrict__ flags, int cap, const int64_t *__restrict__ d_count,
    const int32_t *__restrict__ part, int nb, int direct, int64_t *__restrict__ d_kept,
    int *__restrict__ order) {
    __shared__ int lds_waves[kKeepThreads / kWave];
    __shared__ long long lds_pre[kKeepThreads / kWave][2];
    __shared__ int s_pos[kKeepTile];  // kept from the front, culled from the back
    const int np = live_pairs(cap, d_count);
    const int b = blockIdx.x;
    const int64_t base = (int64_t)b * kKeepTile;
    if (base >= np) {  // uniform: no pair in this block
        if (b == 0 && direct && threadIdx.x == 0) *d_kept = 0;
        return;
    }
    long long prefix = 0;
    if (direct) {
        long long pre = 0, all = 0;
        for (int j = threadIdx.x; j < nb; j += kKeepThreads) {
            const int v = part[j];
            pre += j < b ? v : 0;
            all += v;
        }
#pragma unroll
        for (int o = kWave / 2; o >= 1; o >>= 1) {
            pre += __shfl_xor(pre, o, kWave);
            all += __shfl_xor(all, o, kWave);
        }
        if ((threadIdx.x & (kWave - 1)) == 0) {
            lds_pre[threadIdx.x / kWave][0] = pre;
            lds_pre[threadIdx.x / kWave][1] = all;
        }
        __syncthreads();
        long long tot = 0;
#pragma unroll
        for (int w = 0; w < kKeepThreads / kWave; ++w) {
            prefix += lds_pre[w][0];
            tot += lds_pre[w][1];
        }
        if (b == 0 && threadIdx.x == 0) *d_kept = tot;
    } else {
        prefix = part[b];
    }
    const int i_loc = threadIdx.x * kKeepItems;
    int valid;
    const unsigned m = keep_mask(flags, base + i_loc, np, &valid);
    int kept_blk;
    int kept = scan_detail::block_exclusive(__popc(m), lds_waves, &kept_blk);
    int culled = i_loc - kept;  // culled pairs of the block before this thread's
    for (int k = 0; k < valid; ++k) {
        if ((m >> k) & 1u)
            s_pos[kept++] = (int)(base + i_loc + k);
        else
            s_pos[kKeepTile - 1 - culled++] = (int)(base + i_loc + k);
    }
    __syncthreads();
    const int n_blk = (int)min<int64_t>(kKeepTile, (int64_t)np - base);
    const int culled_blk = n_blk - kept_blk;
    const int64_t culled_before = base - prefix;  // every pair before the block is below np
    for (int j = threadIdx.x; j < kept_blk; j += kKeepThreads) order[prefix + j] = s_pos[j];
    for (int j = threadIdx.x; j < culled_blk; j += kKeepThreads)
        order[np - 1 - culled_before - j] = s_pos[kKeepTile - 1 - j];
}


// Which tiles the wave's pairs lie in (cheap: one coalesced load and ballots).
template <int C>
__device__ __forceinline__ bool bwd_slots(const BwdArgs &a, int64_t p0, BwdLane<C> &L,
                                          uint64_t &starts, int &nslots) {
    const int lane = threadIdx.x;
    const int64_t q = p0 + lane;
    L.p = q < a.n_work ? bwd_pair(a, q) : -1;
    int tile = L.p >= 0 ? a.pair_tiles[L.p] : -1;
    if (tile < 0 || tile >= a.T) tile = -1;
    L.tile = tile;
    L.valid = tile >= 0;
    const int prev_tile = __shfl_up(tile, 1, kWave);
    starts = __ballot(L.valid && (lane == 0 || prev_tile != tile));
    nslots = __popcll(starts);
    const uint64_t upto = lane == kWave - 1 ? ~0ull : ((2ull << lane) - 1);
    L.slot = L.valid ? __popcll(starts & upto) - 1 : -1;
    return nslots > 0;
}

// Shift K of the chained row evaluation of one gate-free pair (pair_moments,
// kRowsChain), or -1 when the pair does not qualify.  With x_u = al p'_u
// (|p'_u| <= 3.5, so x_u^2 <= 12.25 al^2), a_u = 2^E_u * G_u,
// G_u = 2^(-x_u^2 - K) and E_u = sigma2_u + off + x_u^2 + K, linear in u with
// the slope 2 al u_r per column (2 al u_r = 2k (a dx + b dy + c dz) at the row
// centre, the form's x-slope), the chain is exact in binary32 flush-to-zero
// arithmetic (every product below 2^-126 is 0 exactly where the reference's
// gate fails, up to rounding at the threshold) when
//  (a) every G_u >= 2^-125 and <= 1: 2 <= K <= 120 - 12.25 al^2;
//  (b) along each chain (an anchor and three steps) no product before a
//      passing voxel, where E >= -126 + K, falls below 2^-124: K >= 3M + 2
//      with M >= |slope| on every row that can hold a passing voxel;
//  (c) no step or E overflows on any row of the tile, live or dead: the slope
//      stays below 120 over the tile's rows (m_tile), and E <= off + 12.25
//      al^2 + K <= 54 everywhere since sigma2 <= 0.
// M is the least of three bounds on the slope: m_tile; on a row whose gate
// interval (half-width <= sqrt(k2 / Q_xx), k2 = -2 ln2 t2) meets the voxel
// centres, whose peak then lies within 3.5 + sqrt(k2 / Q_xx) of the row
// centre, 2 al^2 times that distance; and over the projection onto (y, z) of
// the gate ellipsoid d^T Q d <= k2, where 2k (b dy + c dz) stays within
// sqrt(k2 w^T Q^-1 w) of 0 (RowForm::r_ell), plus 2 al^2 |mx|.  K is the
// admissible integer nearest -off: E at the Gaussian's peak is then near
// x_u^2, where the exp2 arguments round least.  (Column factors about the
// Gaussian's centre instead, x_u - al mx, step only by the form's coupling
// but carry |x_u - al mx|^2 into E; measured at cfg3 they left ~1.9x as many
// dconics elements outside rel 1e-4 / abs 1e-6 for an N(0,1) vol_grad.)
// Binary32 margins: 1e-3 relative and 0.01 on M.  The terms that depend on
// the Gaussian alone come from its record: k_max = floor(120 - 12.25 al^2),
// m_reach, s_ell = sqrt(k2 r_ell) and rint(-off).
__device__ __forceinline__ float chain_shift(const RowForm &f, float mxl, float k_max,
                                             float m_reach, float s_ell, float kch0) {
    const float a2 = f.al * f.al;
    const float m_tile = 2.0f * f.al * (fabsf(f.tc) + 3.5f * (fabsf(f.be) + fabsf(f.ga)));
    if (!(m_tile < 120.0f)) return -1.0f;
    const float m_ell = 2.0f * a2 * fabsf(mxl) + s_ell;
    const float M = fminf(m_tile, fminf(m_ell, m_reach)) * 1.001f + 0.01f;
    const float k_min = ceilf(3.0f * M) + 2.0f;
    if (!(k_min <= k_max)) return -1.0f;
    return fminf(k_max, fmaxf(k_min, kch0));
}

// The lane's Gaussian (its record), its gate, its offsets from the tile centre
// and, in the deterministic mode, its emission slot.
template <int C>
__device__ __forceinline__ void bwd_gaussian(const BwdArgs &a, BwdLane<C> &L) {
    L.live = L.fast = false;
    L.g = 0;
    L.mxl = L.myl = L.mzl = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) L.I[c] = 0.f;
    L.off = kDeadOffset;
    L.fscale = 0.f;
    L.rf = RowForm{};
    L.kch = -1.0f;
    L.slot_e = -1;
    L.rp = nullptr;
    L.tg = tile_geom(L.valid ? L.tile : 0, a.fx, a.Tx, a.fy, a.Ty, a.D, a.H, a.W);
    if (!L.valid) return;
    const int g = a.ids[L.p];
    L.g = g;
    if ((unsigned)g >= (unsigned)a.n) return;
    const float4 *rp = a.rec + (size_t)g * kBwdRecF4;
    L.rp = rp;
    const float4 r0 = rp[0], r1 = rp[1], r2 = rp[2];
    L.I[0] = r2.z;
#pragma unroll
    for (int c = 1; c < C; ++c) L.I[c] = a.intens[(size_t)g * C + c];
    const TileGeom &tg = L.tg;
    if (a.partial != nullptr) {
        // e = cum[g-1] + ((tz-min.z)*ny + (ty-min.y))*nx + (tx-min.x), the order
        // the pairs were duplicated in; -1 outside [cum[g-1], cum[g]) or past
        // the pair count (as emission_slot_at)
        const float4 r4 = rp[4], r5 = rp[5];
        const int tx = tg.x0 / GSV_TILE, ty = tg.y0 / GSV_TILE, tz = tg.z0 / GSV_TILE;
        const int nx = __float_as_int(r5.x), ny = __float_as_int(r5.y);
        const int64_t base = __float_as_int(r5.z), end = __float_as_int(r5.w);
        const int64_t e = (int64_t)__double_as_longlong(rec_double(r4.z, r4.w)) +
                          ((int64_t)tz * ny + ty) * nx + tx;
        L.slot_e = (e >= base && e < end && e < (int64_t)a.n_isect) ? (int)e : -1;
    }
    const unsigned flags = (unsigned)__float_as_int(r0.w);
    L.off = r1.x;
    L.live = (flags & kRecLive) != 0;
    // A work list holds only pairs the forward's identical test kept, so the
    // test is not repeated for them (a pair it would cull has no passing
    // voxel and yields zero moments either way).
    if (L.live && (flags & kRecBounded) && a.order == nullptr) {
        const float2 c01 = a.conics[3 * g], c23 = a.conics[3 * g + 1], c45 = a.conics[3 * g + 2];
        L.live = may_touch(r0.x, r0.y, r0.z, c01.x, c01.y, c23.x, c23.y, c45.x, c45.y, r2.w,
                           tg.xlo, tg.xhi, tg.ylo, tg.yhi, tg.zlo, tg.zhi);
    }
    if (L.live) {
        L.fast = (flags & kRecFast) != 0;
        // delta = mu - p = (mu - tile centre) - p', p' = local index - 3.5
        L.mxl = r0.x - (float)tg.x0 - 4.0f;
        L.myl = r0.y - (float)tg.y0 - 4.0f;
        L.mzl = r0.z - (float)tg.z0 - 4.0f;
        if (L.fast) {
            // 2^-off of the rounded offset, as make_gate forms it
            L.fscale = __builtin_amdgcn_exp2f(-L.off);
            const float4 r3 = rp[3], r4 = rp[4];
            const float al = r1.w;
            row_centre(al, r2.x, r2.y, rec_double(r3.x, r3.y), rec_double(r3.z, r3.w),
                       rec_double(r4.x, r4.y), L.mxl, L.myl, L.mzl, L.rf);
            const float k_max = floorf(120.0f - 12.25f * (al * al));
            L.kch = chain_shift(L.rf, L.mxl, k_max, r1.z, r1.y, rintf(-L.off));
        }
    }
}

// The gate of the lane's Gaussian from its intensities (the exact path's
// shift, half-width and scale), as make_gate takes it; make_gate(0) for a lane
// without a Gaussian.
template <int C>
__device__ __forceinline__ Gate lane_gate(const BwdLane<C> &L) {
    float mean = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) mean += L.I[c];
    mean /= (float)C;
    return make_gate(mean);
}

// Exponent e such that m * 2^e lies in [2^(kGradScaleExp-1), 2^kGradScaleExp);
// 0 for m = 0, infinite or NaN.
__device__ __forceinline__ int grad_scale_exp(float m) {
    if (!(m > 0.f && m <= FLT_MAX)) return 0;
    int e;
    (void)frexpf(m, &e);
    return kGradScaleExp - e;
}

// One staged row of the backward's source gradient: x = x0 .. x0+nx-1 of one
// (y, z), C channels, at element offset `off`.  With the fused L1 sign bytes
// the value is sc * sgn, plus vol_grad when that is given
// too; otherwise it is vol_grad.  Full rows at a suitable alignment are read
// with vector loads (one 8-byte load per 8 sign bytes, float4 for vol_grad).
template <int C>
__device__ __forceinline__ void load_grad_row(const BwdArgs &a, int64_t off, int nx, float sc,
                                              float (&v)[GSV_TILE * C]) {
    constexpr int kN = GSV_TILE * C;
    if (a.l1_sgn != nullptr) {
        const int8_t *sg = a.l1_sgn + off;
        if (nx == GSV_TILE && ((uintptr_t)sg & 7) == 0) {
            uint32_t w[kN / 4];
#pragma unroll
            for (int q = 0; q < kN / 8; ++q) {
                const uint2 t = reinterpret_cast<const uint2 *>(sg)[q];
                w[2 * q] = t.x;
                w[2 * q + 1] = t.y;
            }
#pragma unroll
            for (int q = 0; q < kN / 4; ++q)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    v[4 * q + b] = sc * (float)(int8_t)(w[q] >> (8 * b));
        } else {
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u)
                if (u < nx)
#pragma unroll
                    for (int c = 0; c < C; ++c) v[u * C + c] = sc * (float)sg[u * C + c];
        }
        if (a.vol_grad != nullptr) {
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u)
                if (u < nx)
#pragma unroll
                    for (int c = 0; c < C; ++c) v[u * C + c] += a.vol_grad[off + u * C + c];
        }
        return;
    }
    const float *src = a.vol_grad + off;
    if (nx == GSV_TILE && ((uintptr_t)src & 15) == 0) {
#pragma unroll
        for (int q = 0; q < kN / 4; ++q) {
            const float4 t = reinterpret_cast<const float4 *>(src)[q];
            v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < GSV_TILE; ++u)
            if (u < nx)
#pragma unroll
                for (int c = 0; c < C; ++c) v[u * C + c] = src[u * C + c];
    }
}

// One group of up to K tiles (slots g0 .. g0+K-1): stage them in LDS (lane =
// row), accumulate each in-group lane's moments against its own tile's rows,
// and write those lanes' gradients.  Lanes outside the group evaluate a zero
// form at the dead offset and write nothing.
template <int C, int K>
__device__ __forceinline__ void bwd_group(const BwdArgs &a, const BwdLane<C> &L, uint64_t starts,
                                          int g0, bool wave_fast, bool any_live, float4 *s_g) {
    constexpr int kRowF4 = 2 * C;              // float4 per staged row
    constexpr int kSlot = kWave * kRowF4 + 1;  // +16 B: slots start on different banks
    const int lane = threadIdx.x;
    const bool mine = L.valid && L.slot >= g0 && L.slot < g0 + K;
    const bool in_grp = mine && L.live;
    Moments<C> M;
    M.S0 = M.Sx = M.Sy = M.Sz = 0.f;
    M.Sxx = M.Sxy = M.Sxz = M.Syy = M.Syz = M.Szz = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) M.dI[c] = 0.f;
    int gexp = 0;  // vol_grad of the group's tiles is staged as g * 2^gexp
    if (any_live) {
        uint64_t rest = starts;
        for (int k = 0; k < g0; ++k) rest &= rest - 1;  // skip earlier groups' tiles
        // the group's tiles; the slots past them are read by no lane, so they
        // are neither staged nor rescaled
        const int ntile = min(K, __popcll(rest));
        const int y_l = lane & 7, z_l = lane >> 3;
        // fused L1 (torch's l1_loss, mean): dL/dv = sgn(v - t) * (dL / numel).  The
        // division is a multiply by the binary32 reciprocal, as torch's division
        // by a host scalar does, so the bits agree.  Without another incoming
        // volume gradient every staged value is 0 or +-sc, so the group's scale
        // follows from |sc| alone and is applied to sc up front (exactly).
        const bool prescaled = a.l1_sgn != nullptr && a.vol_grad == nullptr;
        float sc = 0.f;
        if (a.l1_sgn != nullptr) {
            sc = *a.l1_grad * (1.0f / a.l1_numel);
            if (prescaled && wave_fast) {
                gexp = grad_scale_exp(fabsf(sc));
                sc = ldexpf(sc, gexp);
            }
        }
        float mx = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if (k >= ntile) break;
            float v[GSV_TILE * C];
#pragma unroll
            for (int i = 0; i < GSV_TILE * C; ++i) v[i] = 0.f;
            if (rest) {
                const int first = __builtin_ctzll(rest);
                rest &= rest - 1;
                // the tile's origin, read from the (valid) lane that starts its run
                const int x0 = __builtin_amdgcn_readlane(L.tg.x0, first);
                const int y = __builtin_amdgcn_readlane(L.tg.y0, first) + y_l;
                const int z = __builtin_amdgcn_readlane(L.tg.z0, first) + z_l;
                if (y < a.H && z < a.D) {
                    const int64_t off = (((int64_t)z * a.H + y) * a.W + x0) * C;
                    const int nx = min(GSV_TILE, a.W - x0);
                    load_grad_row<C>(a, off, nx, sc, v);
                }
            }
            if (!prescaled) {
#pragma unroll
                for (int i = 0; i < GSV_TILE * C; ++i) mx = fmaxf(mx, fabsf(v[i]));
            }
#pragma unroll
            for (int q = 0; q < kRowF4; ++q)
                s_g[k * kSlot + lane * kRowF4 + q] =
                    make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        }
        if (wave_fast && !prescaled) {  // one power-of-two scale for the group, applied in LDS
#pragma unroll
            for (int o = kWave / 2; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
            gexp = grad_scale_exp(mx);
            if (gexp != 0) {
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    if (k >= ntile) break;
#pragma unroll
                    for (int q = 0; q < kRowF4; ++q) {
                        float4 &t4 = s_g[k * kSlot + lane * kRowF4 + q];
                        t4 = make_float4(ldexpf(t4.x, gexp), ldexpf(t4.y, gexp),
                                         ldexpf(t4.z, gexp), ldexpf(t4.w, gexp));
                    }
                }
            }
        }
        __syncthreads();
        const int my = in_grp ? L.slot - g0 : 0;
        const float gx = in_grp ? L.mxl : 0.f, gy = in_grp ? L.myl : 0.f, gz = in_grp ? L.mzl : 0.f;
        if (wave_fast) {
            // lanes outside the group: a zero form (zero coefficients) at the dead offset
            const RowForm rf = in_grp ? L.rf : RowForm{};
            const float off = in_grp ? L.off : kDeadOffset;
            const float kshift = in_grp ? L.kch : 2.0f;
            float Gt[GSV_TILE];
#pragma unroll
            for (int u = 0; u < GSV_TILE; ++u) Gt[u] = 1.0f;
            if (a.chain && __all(kshift >= 0.f)) {
                if (in_grp) {  // the Gaussian's column factors (read here, not held across the staging)
                    const float4 r6 = L.rp[6], r7 = L.rp[7];
                    Gt[0] = r6.x; Gt[1] = r6.y; Gt[2] = r6.z; Gt[3] = r6.w;
                    Gt[4] = r7.x; Gt[5] = r7.y; Gt[6] = r7.z; Gt[7] = r7.w;
                }
                pair_moments<C, kRowsChain>(s_g + my * kSlot, gx, gy, gz, rf, 0.f, 0.f, 0.f, 0.f, 0.f,
                                            0.f, 0.f, off, kshift, Gt, L.I, M);
            } else {
                pair_moments<C, kRowsForm>(s_g + my * kSlot, gx, gy, gz, rf, 0.f, 0.f, 0.f, 0.f, 0.f,
                                           0.f, 0.f, off, 0.f, Gt, L.I, M);
            }
        } else {
            // lanes outside the group: a zero form, never inside the gate (|s| <= -1)
            float2 c01 = make_float2(0.f, 0.f), c23 = c01, c45 = c01;
            if (in_grp) {
                c01 = a.conics[3 * L.g];
                c23 = a.conics[3 * L.g + 1];
                c45 = a.conics[3 * L.g + 2];
            }
            const Gate gt = lane_gate(L);
            const float A2 = in_grp ? -0.5f * kLog2e * c01.x : 0.f, Bn = in_grp ? -kLog2e * c01.y : 0.f;
            const float Cn = in_grp ? -kLog2e * c23.x : 0.f, Dn = in_grp ? -0.5f * kLog2e * c23.y : 0.f;
            const float En = in_grp ? -kLog2e * c45.x : 0.f, Fn = in_grp ? -0.5f * kLog2e * c45.y : 0.f;
            const float Gt[GSV_TILE] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};  // unused
            pair_moments<C, kRowsExact>(s_g + my * kSlot, gx, gy, gz, RowForm{}, A2, Bn, Cn, Dn, En,
                                        Fn, gt.shift, in_grp ? gt.half : -1.f, 0.f, Gt, L.I, M);
        }
        __syncthreads();  // a later group restages the slots
    }
    if (!mine) return;
    // sigma-gradient weight per unit of h (alpha = scale * a) as ws * 2^we: the
    // 2^-gexp and 2^-off factors stay in the exponent, so each product below is
    // a binary32 number in range (gate-free: ws < 1, I < 2^54, moments < 2^45),
    // and ldexpf applies them exactly
    float ws = 0.f;
    int we = 0;
    if (L.live) {
        if (wave_fast) {
            ws = frexpf(L.fscale, &we);
            we -= gexp;
        } else {
            ws = lane_gate(L).scale;
        }
    }
    const float w = (C == 1) ? ws * L.I[0] : ws;
    float out[9 + C];
    out[0] = ldexpf(-w * M.Sxx, we - 1);
    out[1] = ldexpf(-w * M.Sxy, we);
    out[2] = ldexpf(-w * M.Sxz, we);
    out[3] = ldexpf(-w * M.Syy, we - 1);
    out[4] = ldexpf(-w * M.Syz, we);
    out[5] = ldexpf(-w * M.Szz, we - 1);
    // dpos = Q (-w S): the deterministic mode stores -w S and k_pair_reduce
    // applies the conic once per Gaussian to the binary64 sum (linear, so the
    // same gradient, with one rounding of Q S instead of one per pair); the
    // atomic mode applies it here
    if (a.partial != nullptr) {
        out[6] = ldexpf(-w * M.Sx, we);
        out[7] = ldexpf(-w * M.Sy, we);
        out[8] = ldexpf(-w * M.Sz, we);
    } else {
        // read again rather than held across the loop (zero without a Gaussian)
        float2 q01 = make_float2(0.f, 0.f), q23 = q01, q45 = q01;
        if ((unsigned)L.g < (unsigned)a.n && L.valid) {
            q01 = a.conics[3 * L.g];
            q23 = a.conics[3 * L.g + 1];
            q45 = a.conics[3 * L.g + 2];
        }
        out[6] = ldexpf(-w * fmaf(q01.x, M.Sx, fmaf(q01.y, M.Sy, q23.x * M.Sz)), we);
        out[7] = ldexpf(-w * fmaf(q01.y, M.Sx, fmaf(q23.y, M.Sy, q45.x * M.Sz)), we);
        out[8] = ldexpf(-w * fmaf(q23.x, M.Sx, fmaf(q45.x, M.Sy, q45.y * M.Sz)), we);
    }
    if (C == 1) {
        out[9] = ldexpf(ws * M.S0, we);
    } else {
#pragma unroll
        for (int c = 0; c < C; ++c) out[9 + c] = ldexpf(ws * M.dI[c], we);
    }
    const int g = L.g;
    if (a.partial != nullptr) {
        // Deterministic path: this pair's partial goes to its emission slot
        const int64_t e = L.slot_e;
        if (e >= 0) {
            float *dst = a.partial + e * (9 + C);
#pragma unroll
            for (int q = 0; q < 9 + C; ++q) dst[q] = out[q];
        }
    } else if (L.live) {
        float *dc = a.dconic + 6 * (size_t)g;
#pragma unroll
        for (int q = 0; q < 6; ++q) unsafeAtomicAdd(dc + q, out[q]);
        float *dp = a.dpos + 4 * (size_t)g;
#pragma unroll
        for (int q = 0; q < 3; ++q) unsafeAtomicAdd(dp + q, out[6 + q]);
        float *di = a.dint + (size_t)C * g;
#pragma unroll
        for (int c = 0; c < C; ++c) unsafeAtomicAdd(di + c, out[9 + c]);
    }
}

// The zero partials of the pairs the forward culled, spread over the W work
// waves: wave wv writes those of culled items [wv*c, (wv+1)*c), c =
// ceil(culled / W), one lane per pair.  culled_slot looks up one item's slot
// (-1: none); the kernel looks up each lane's first item before its own work
// and writes the zeros after it, so those loads overlap the work.
__device__ __forceinline__ int64_t culled_slot(const BwdArgs &a, int64_t q) {
    const int p = a.order[a.n_isect - 1 - q];
    const int t = a.pair_tiles[p];
    if (t < 0 || t >= a.T) return -1;
    return emission_slot(a.ids[p], t, a);
}

template <int C>
__device__ __forceinline__ void zero_partial(const BwdArgs &a, int64_t e) {
    float *dst = a.partial + e * (9 + C);
#pragma unroll
    for (int k = 0; k < 9 + C; ++k) dst[k] = 0.f;
}

// One wave per 64 consecutive (tile, Gaussian) pairs of the sorted list (or of
// the work list of kept pairs), lane = pair, so no lane idles except in the
// last wave.  The wave stages the first K tiles its pairs span (lane = row;
// each lane reads its own tile's rows); the pairs of further tiles are left to
// k_vox_bwd_rest.  At C = 2 and 3 the kernel fits 128 VGPRs (4 waves per
// SIMD), but left free the compiler's schedule for C = 2, K = 6 and C = 3,
// K = 4 took all 256 and spilled into AGPRs (1 wave per SIMD): the bound
// holds those two to the others' occupancy.  C = 1 (106 VGPRs) and C = 4
// (3 waves) take the compiler's own choice.  C = 3, K = 6 stages 36,960 bytes,
// which LDS holds to one wave per SIMD: there the bound only caps the
// registers (128 VGPRs, no AGPRs), and the compiler's note that it missed the
// occupancy target is silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
template <int C, int K>
__global__ __launch_bounds__(kWave)
__attribute__((amdgpu_waves_per_eu(C == 2 || C == 3 ? 2 : 1, 8))) void k_vox_bwd(BwdArgs a) {
    __shared__ float4 s_g[K * (kWave * 2 * C + 1)];
    bwd_counts(a);
    // XCD slabs sized by the live wave count (the grid may be sized for a
    // larger capacity), so every XCD gets an equal share; blocks past the
    // slabs would alias waves of other blocks and leave.  With a work list at
    // least one wave runs, for the culled pairs' zeros.
    const bool zeros = a.order != nullptr && a.partial != nullptr;
    const int64_t waves = ((int64_t)a.n_work + kWave - 1) / kWave;
    const int64_t W = zeros ? max<int64_t>(waves, 1) : waves;
    const int64_t per = xcd_per(W);
    if ((int64_t)(blockIdx.x / kXcds) >= per) return;
    const int64_t wv = xcd_remap(blockIdx.x, per);
    int64_t zq = 0, zq1 = 0, ze = -1;  // this lane's culled items [zq, zq1), step kWave
    if (zeros) {
        const int64_t culled = (int64_t)a.n_isect - a.n_work;
        const int64_t c = culled > 0 ? (culled + W - 1) / W : 0;
        zq = wv * c + threadIdx.x;
        zq1 = min<int64_t>(culled, (wv + 1) * c);
        if (zq < zq1) ze = culled_slot(a, zq);
    }
    const int64_t p0 = wv * kWave;
    if (p0 < a.n_work) {
        BwdLane<C> L;
        uint64_t starts;
        int nslots;
        const bool slots = bwd_slots(a, p0, L, starts, nslots);
        if (threadIdx.x == 0) a.rest_flag[wv] = slots && nslots > K;
        if (slots) {
            bwd_gaussian(a, L);
            // one wave-uniform choice: gate-free unless a live lane needs the exact gate
            const bool wave_fast = __all(!L.live || L.fast);
            const bool any_live = __any(L.live);
            if (any_live || a.partial != nullptr)
                bwd_group<C, K>(a, L, starts, 0, wave_fast, any_live, s_g);
        }
    }
    if (ze >= 0) zero_partial<C>(a, ze);
    for (int64_t q = zq + kWave; q < zq1; q += kWave) {
        const int64_t e = culled_slot(a, q);
        if (e >= 0) zero_partial<C>(a, e);
    }
}
#pragma clang diagnostic pop

// The pairs that k_vox_bwd left: those of the waves spanning more than K tiles,
// in groups of K tiles after the first.  A fixed grid of kRestBlocks
// workgroups; workgroup b reads the flags of the waves b, b + G, b + 2G, ...
// (G = the grid size) 64 at a time, so the waves to process (many in a sparse
// scene, none in most dense ones) spread over the whole grid.
constexpr int kRestBlocks = 512;

template <int C, int K>
__global__ __launch_bounds__(kWave) void k_vox_bwd_rest(BwdArgs a) {
    __shared__ float4 s_g[K * (kWave * 2 * C + 1)];
    bwd_counts(a);
    const int64_t waves = ((int64_t)a.n_work + kWave - 1) / kWave;
    const int64_t G = gridDim.x;
    for (int64_t base = blockIdx.x; base < waves; base += G * kWave) {
        const int64_t w = base + (int64_t)threadIdx.x * G;
        const bool more = w < waves && a.rest_flag[w] != 0;
        for (uint64_t m = __ballot(more); m; m &= m - 1) {
            const int64_t p0 = (base + (int64_t)__builtin_ctzll(m) * G) * kWave;
            BwdLane<C> L;
            uint64_t starts;
            int nslots;
            if (!bwd_slots(a, p0, L, starts, nslots) || nslots <= K) continue;
            bwd_gaussian(a, L);
            const bool wave_fast = __all(!L.live || L.fast);
            const bool any_live = __any(L.live);
            if (!any_live && a.partial == nullptr) continue;
            for (int g0 = K; g0 < nslots; g0 += K)
                bwd_group<C, K>(a, L, starts, g0, wave_fast, any_live, s_g);
        }
    }
}

// Deterministic reduction of the per-pair partials: one 16-lane DPP row per
// Gaussian g.  Lane r of the row sums slots cum[g-1] + r, + r + 16, ... of
// [cum[g-1], cum[g]) (a row's loads cover 16 consecutive slots), then a fixed
// row_shr 1, 2, 4, 8 scan adds the 16 lane sums; all in binary64, lane 15
// writes every output element, dpos as the conic times the summed -w S of the
// partials.  DPP keeps the cross-lane sums on the VALU (an xor-shuffle
// butterfly goes through the LDS crossbar, 2 ops per double).
constexpr int kRowLanes = 16;
constexpr int kReduceThreads = 256;

template <int kCtrl>
__device__ __forceinline__ double row_shr(double x) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(x), kCtrl, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(x), kCtrl, 0xf, 0xf, true);
    return __hiloint2double(hi, lo);
}

template <int kCtrl>
__device__ __forceinline__ float row_shr_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, true));
}

// Inclusive scan within each 16-lane row; lane 15 ends with the row total.
__device__ __forceinline__ double row_total(double x) {
    x += row_shr<0x111>(x);
    x += row_shr<0x112>(x);
    x += row_shr<0x114>(x);
    x += row_shr<0x118>(x);
    return x;
}

template <int C>
__global__ __launch_bounds__(kReduceThreads) void k_pair_reduce(
    int n, int cap, const int64_t *__restrict__ d_count, const float4 *__restrict__ rec,
    const float *__restrict__ partial, const float *__restrict__ conics,
    float *__restrict__ dpos, float *__restrict__ dconic, float *__restrict__ dint) {
    const int n_isect = live_pairs(cap, d_count);
    constexpr int F = 9 + C;
    const int r = threadIdx.x & (kRowLanes - 1);
    const int g = (int)(((int64_t)blockIdx.x * kReduceThreads + threadIdx.x) / kRowLanes);
    int64_t b = 0, e = 0;
    // the conic for dpos = Q T: lane r < 6 of the row reads element r, before
    // the partials so that its latency overlaps them (one load for the wave)
    float qv = 0.f;
    if (g < n) {  // rows past n reduce zeros; every lane stays for the DPP steps
        // [cum[g-1], cum[g]) from the Gaussian's record, which the backward just read
        const float4 r5 = rec[(size_t)g * kBwdRecF4 + 5];
        b = max(0, __float_as_int(r5.z));
        e = min<int64_t>(__float_as_int(r5.w), n_isect);
        if (r < 6) qv = conics[6 * (size_t)g + r];
    }
    double acc[F];
#pragma unroll
    for (int q = 0; q < F; ++q) acc[q] = 0.0;
    for (int64_t k = b + r; k < e; k += kRowLanes) {
        const float *src = partial + k * F;
#pragma unroll
        for (int q = 0; q < F; ++q) acc[q] += (double)src[q];
    }
#pragma unroll
    for (int q = 0; q < F; ++q) acc[q] = row_total(acc[q]);
    // conic element k from lane k to lane 15 of the row (row_shr 15 - k)
    const float qa = row_shr_f32<0x11f>(qv), qb = row_shr_f32<0x11e>(qv);
    const float qc = row_shr_f32<0x11d>(qv), qd = row_shr_f32<0x11c>(qv);
    const float qe = row_shr_f32<0x11b>(qv), qf = row_shr_f32<0x11a>(qv);
    if (r != kRowLanes - 1 || g >= n) return;
    float2 *dc = reinterpret_cast<float2 *>(dconic + 6 * (size_t)g);
    dc[0] = make_float2((float)acc[0], (float)acc[1]);
    dc[1] = make_float2((float)acc[2], (float)acc[3]);
    dc[2] = make_float2((float)acc[4], (float)acc[5]);
    // dpos = Q T, T = the summed -w S of the pairs (binary64); a Gaussian without
    // pairs gets zeros whatever its conic
    float4 dp = make_float4(0.f, 0.f, 0.f, 0.f);
    if (b < e) {
        const double a = qa, bb = qb, c = qc, d = qd, ee = qe, f = qf;
        dp.x = (float)(a * acc[6] + bb * acc[7] + c * acc[8]);
        dp.y = (float)(bb * acc[6] + d * acc[7] + ee * acc[8]);
        dp.z = (float)(c * acc[6] + ee * acc[7] + f * acc[8]);
    }
    reinterpret_cast<float4 *>(dpos)[g] = dp;
#pragma unroll
    for (int c = 0; c < C; ++c) dint[(size_t)C * g + c] = (float)acc[9 + c];
}

struct BwdLayout {
    size_t rec, tiles, partial, order, part, kept, rest, end;
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// the per-Gaussian records (n * 128 bytes), the pair -> tile map (n_isect
// ints; unused when the caller passes the binning's sorted keys), the per-pair
// partials in pairs mode, the work list of the culled mode (order, the
// per-block counts and the kept count), then the backward's per-wave rest
// flags.
BwdLayout bwd_layout(int64_t n, int64_t n_isect, int channels, bool pairs) {
    BwdLayout L{};
    size_t off = 0;
    L.rec = off; off += align256((size_t)imax64(n, 1) * kBwdRecF4 * sizeof(float4));
    L.tiles = off; off += align256((size_t)imax64(n_isect, 1) * 4);
    L.partial = off;
    if (pairs) off += align256((size_t)n_isect * (9 + channels) * 4);
    L.order = off; off += align256((size_t)imax64(n_isect, 1) * 4);
    L.part = off; off += align256((size_t)((n_isect + kKeepTile - 1) / kKeepTile + 1) * 4);
    L.kept = off; off += 256;
    L.rest = off; off += align256((size_t)((imax64(n_isect, 1) + kWave - 1) / kWave));
    L.end = off;
    return L;
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace gsv

namespace gsv {
namespace {

// Forward; with `target`, also the L1 loss mean|volume - target| into *loss
// (tile_loss: T floats of scratch) and sgn(volume - target) into sgn.
int voxelize_fwd_impl(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                      int64_t num_intersects, const int32_t *ids, const int32_t *tile_bins,
                      const float *pos3d_radii, const float *conics, const float *intensities,
                      float *volume, const float *target, float *tile_loss, int8_t *sgn,
                      float *loss, uint8_t *pair_live, hipStream_t s) {
    if (channels < 1 || channels > GSV_MAX_CHANNELS) return GSV_ERR_UNSUPPORTED_CHANNELS;
    if (n < 0 || D <= 0 || H <= 0 || W <= 0 || !volume || !tile_bins) return GSV_ERR_INVALID_ARGUMENT;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    const int64_t T = (int64_t)Tx * Ty * Tz;
    const int64_t vox = (int64_t)D * H * W;
    if (vox * channels > ((int64_t)1 << 40) || T > INT32_MAX || num_intersects > INT32_MAX)
        return GSV_ERR_SIZE_OVERFLOW;
    const bool empty = num_intersects <= 0 || n == 0;
    if (empty && !target) return fill_zero_u32(volume, vox * channels, s);
    if (!empty && (!ids || !pos3d_radii || !conics || !intensities)) return GSV_ERR_INVALID_ARGUMENT;
    if (!empty && (!aligned(pos3d_radii, 16) || !aligned(conics, 8))) return GSV_ERR_INVALID_ARGUMENT;
    // an empty list still runs the kernel for the loss: every tile range is empty
    const int ni = empty ? 0 : (int)num_intersects;
    const dim3 grid((unsigned)xcd_runs_grid(T)), block(kWave);
    int wave_cap = 0;
    uint64_t *wave_rec = wave_timeline_buffer(&wave_cap);
    {
        KernelTimer timer(kTimedVoxFwd, s);
#define GSV_VF(CH)                                                                                 \
    hipLaunchKernelGGL(k_vox_fwd<CH>, grid, block, 0, s, D, H, W, Tx, Ty, T, n, ni, ids,           \
                       reinterpret_cast<const int2 *>(tile_bins),                                  \
                       reinterpret_cast<const float4 *>(pos3d_radii),                              \
                       reinterpret_cast<const float2 *>(conics), intensities, volume, target,      \
                       tile_loss, sgn, pair_live, wave_rec, wave_cap)
        switch (channels) {
            case 1: GSV_VF(1); break;
            case 2: GSV_VF(2); break;
            case 3: GSV_VF(3); break;
            default: GSV_VF(4); break;
        }
#undef GSV_VF
    }
    if (int st = check_launch()) return st;
    if (target) {
        hipLaunchKernelGGL(k_loss_finish, dim3(1), dim3(kFinishThreads), 0, s, tile_loss, T,
                           (double)vox * channels, loss);
        return check_launch();
    }
    return GSV_OK;
}

// Backward from vol_grad, or (l1_sgn set) from the fused L1 loss: dL/dv =
// sgn(volume - target) * (*l1_grad / numel) + vol_grad (vol_grad optional),
// l1_sgn being the signs gsv_voxelize_fwd_l1 stored.
int voxelize_bwd_impl(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                      int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                      const int32_t *tile_bins, const float *pos3d_radii, const float *conics,
                      const float *intensities, const float *vol_grad, const int8_t *l1_sgn,
                      const float *l1_grad, const int32_t *tile_min,
                      const int32_t *tile_max, const int32_t *cum_tiles_hit,
                      const int32_t *tiles_sorted, const int64_t *count_dev,
                      const uint8_t *pair_live, float *dpos3d_radii, float *dconics,
                      float *dintensities, int32_t variant, void *workspace,
                      size_t workspace_bytes, hipStream_t s) {
    if (channels < 1 || channels > GSV_MAX_CHANNELS) return GSV_ERR_UNSUPPORTED_CHANNELS;
    if (n < 0 || D <= 0 || H <= 0 || W <= 0 || (variant != 0 && variant != 1))
        return GSV_ERR_INVALID_ARGUMENT;
    if (n == 0) return GSV_OK;
    if (!dpos3d_radii || !dconics || !dintensities) return GSV_ERR_INVALID_ARGUMENT;
    const bool pairs = tile_min && tile_max && cum_tiles_hit;
    if (!pairs && (tile_min || tile_max || cum_tiles_hit)) return GSV_ERR_INVALID_ARGUMENT;
    if (num_intersects <= 0 || !pairs) {
        if (int st = fill_zero_u32(dpos3d_radii, 4 * (int64_t)n, s)) return st;
        if (int st = fill_zero_u32(dconics, 6 * (int64_t)n, s)) return st;
        if (int st = fill_zero_u32(dintensities, (int64_t)channels * n, s)) return st;
    }
    if (num_intersects <= 0) return GSV_OK;
    const bool l1 = l1_sgn != nullptr;
    if (!gaussian_ids_sorted || !tile_bins || !pos3d_radii || !conics || !intensities ||
        (!l1 && !vol_grad) || (l1 && !l1_grad))
        return GSV_ERR_INVALID_ARGUMENT;
    if (!aligned(pos3d_radii, 16) || !aligned(conics, 8) || !aligned(dpos3d_radii, 16) ||
        !aligned(dconics, 8))
        return GSV_ERR_INVALID_ARGUMENT;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    const int64_t T = (int64_t)Tx * Ty * Tz;
    if (T > INT32_MAX || num_intersects > INT32_MAX) return GSV_ERR_SIZE_OVERFLOW;
    const BwdLayout L = bwd_layout(n, num_intersects, channels, pairs);
    if (!workspace || workspace_bytes < L.end) return GSV_ERR_WORKSPACE_TOO_SMALL;
    char *ws = static_cast<char *>(workspace);
    const int *pair_tiles = tiles_sorted;
    float *partial = pairs ? reinterpret_cast<float *>(ws + L.partial) : nullptr;
    const int ni = (int)num_intersects;
    if (!pair_tiles) {  // rebuild the pair -> tile map from the tile ranges
        int *own = reinterpret_cast<int *>(ws + L.tiles);
        hipLaunchKernelGGL(k_pair_tiles, dim3((unsigned)T), dim3(kWave), 0, s,
                           reinterpret_cast<const int2 *>(tile_bins), ni, own);
        if (int st = check_launch()) return st;
        pair_tiles = own;
    }
    // the per-Gaussian records: in the work list's count launch when there is
    // one, else a launch of their own
    PrepArgs prep;
    prep.n = n;
    prep.pos_radii = reinterpret_cast<const float4 *>(pos3d_radii);
    prep.conics = reinterpret_cast<const float2 *>(conics);
    prep.intens = intensities;
    prep.tile_min = tile_min; prep.tile_max = tile_max; prep.cum = cum_tiles_hit;
    prep.rec = reinterpret_cast<float4 *>(ws + L.rec);
    const int nprep = (int)((n + kPrepThreads - 1) / kPrepThreads);
    if (!pair_live) {
        const dim3 pgrid((unsigned)nprep), pblock(kPrepThreads);
        switch (channels) {
            case 1: hipLaunchKernelGGL(k_bwd_prep<1>, pgrid, pblock, 0, s, prep); break;
            case 2: hipLaunchKernelGGL(k_bwd_prep<2>, pgrid, pblock, 0, s, prep); break;
            case 3: hipLaunchKernelGGL(k_bwd_prep<3>, pgrid, pblock, 0, s, prep); break;
            default: hipLaunchKernelGGL(k_bwd_prep<4>, pgrid, pblock, 0, s, prep); break;
        }
        if (int st = check_launch()) return st;
    }
    const int *order = nullptr;
    const int64_t *d_work = nullptr;
    if (pair_live) {  // the work list of the pairs the forward kept
        if (!aligned(pair_live, 16)) return GSV_ERR_INVALID_ARGUMENT;
        int *ord = reinterpret_cast<int *>(ws + L.order);
        int32_t *part = reinterpret_cast<int32_t *>(ws + L.part);
        int64_t *kept = reinterpret_cast<int64_t *>(ws + L.kept);
        const int64_t nb = (num_intersects + kKeepTile - 1) / kKeepTile;
        const int direct = nb <= scan_detail::kDirectBlocks ? 1 : 0;
        const dim3 kgrid((unsigned)(nprep + nb)), kblock(kKeepThreads);
#define GSV_KC(CH)                                                                                 \
    hipLaunchKernelGGL(k_keep_count<CH>, kgrid, kblock, 0, s, pair_live, ni, count_dev, part,      \
                       nprep, prep)
        switch (channels) {
            case 1: GSV_KC(1); break;
            case 2: GSV_KC(2); break;
            case 3: GSV_KC(3); break;
            default: GSV_KC(4); break;
        }
#undef GSV_KC
        if (int st = check_launch()) return st;
        if (!direct) {
            hipLaunchKernelGGL(scan_detail::k_scan_block_sums, dim3(1),
                               dim3(scan_detail::kSumsThreads), 0, s, part, nb, kept, nullptr);
            if (int st = check_launch()) return st;
        }
        hipLaunchKernelGGL(k_keep_order, dim3((unsigned)nb), dim3(kKeepThreads), 0, s, pair_live,
                           ni, count_dev, part, (int)nb, direct, kept, ord);
        if (int st = check_launch()) return st;
        order = ord;
        d_work = kept;
    }
    const int64_t waves = (num_intersects + kWave - 1) / kWave;
    const int64_t per = xcd_per(waves);
    const dim3 grid((unsigned)(kXcds * per)), block(kWave);
    const float numel = (float)((int64_t)D * H * W * channels);
    BwdArgs args;
    args.D = D; args.H = H; args.W = W; args.Tx = Tx; args.Ty = Ty; args.n = n; args.n_isect = ni;
    args.fx = make_fastdiv((uint32_t)Tx);
    args.fy = make_fastdiv((uint32_t)Ty);
    args.chain = bwd_chains_enabled() ? 1 : 0;
    args.T = T;
    args.ids = gaussian_ids_sorted; args.pair_tiles = pair_tiles;
    args.pos_radii = reinterpret_cast<const float4 *>(pos3d_radii);
    args.conics = reinterpret_cast<const float2 *>(conics);
    args.intens = intensities; args.vol_grad = vol_grad;
    args.l1_sgn = l1_sgn; args.l1_grad = l1_grad; args.l1_numel = numel;
    args.dpos = dpos3d_radii; args.dconic = dconics; args.dint = dintensities;
    args.tile_min = tile_min; args.tile_max = tile_max; args.cum = cum_tiles_hit;
    args.rec = reinterpret_cast<const float4 *>(ws + L.rec);
    args.partial = partial;
    args.d_count = count_dev;
    args.order = order;
    args.d_work = d_work;
    args.n_work = 0;
    args.rest_flag = reinterpret_cast<uint8_t *>(ws + L.rest);
#define GSV_VB(CH)                                                                                  \
    {                                                                                               \
        KernelTimer timer(kTimedVoxBwd, s);                                                         \
        if (very_sparse) {                                                                          \
            hipLaunchKernelGGL((k_vox_bwd<CH, kStageTilesVerySparse<CH>>), grid, block, 0, s,       \
                               args);                                                               \
            if (int st = check_launch()) return st;                                                 \
            hipLaunchKernelGGL((k_vox_bwd_rest<CH, kStageTilesVerySparse<CH>>),                     \
                               dim3(kRestBlocks), block, 0, s, args);                               \
        } else if (sparse) {                                                                        \
            hipLaunchKernelGGL((k_vox_bwd<CH, kStageTilesSparse<CH>>), grid, block, 0, s, args);   \
            if (int st = check_launch()) return st;                                                 \
            hipLaunchKernelGGL((k_vox_bwd_rest<CH, kStageTilesSparse<CH>>), dim3(kRestBlocks),     \
                               block, 0, s, args);                                                  \
        } else {                                                                                    \
            hipLaunchKernelGGL((k_vox_bwd<CH, kStageTiles<CH>>), grid, block, 0, s, args);         \
            if (int st = check_launch()) return st;                                                 \
            hipLaunchKernelGGL((k_vox_bwd_rest<CH, kStageTiles<CH>>), dim3(kRestBlocks), block, 0, \
                               s, args);                                                            \
        }                                                                                           \
    }                                                                                               \
    if (int st = check_launch()) return st;                                                         \
    if (pairs) {                                                                                    \
        KernelTimer timer(kTimedPairReduce, s);                                                     \
        hipLaunchKernelGGL(k_pair_reduce<CH>,                                                      \
                           dim3((unsigned)(((int64_t)n * kRowLanes + kReduceThreads - 1) /          \
                                           kReduceThreads)),                                        \
                           dim3(kReduceThreads), 0, s, n, ni, count_dev, args.rec, partial,        \
                           conics, dpos3d_radii, dconics,                                           \
                           dintensities);                                                           \
    }
    // pairs per tile from the count the grids are sized for (an upper bound
    // when the live count is on the device)
    const bool sparse = num_intersects < kSparsePairs * T;
    const bool very_sparse = num_intersects < kVerySparsePairs * T;
    switch (channels) {
        case 1: { GSV_VB(1) break; }
        case 2: { GSV_VB(2) break; }
        case 3: { GSV_VB(3) break; }
        default: { GSV_VB(4) break; }
    }
#undef GSV_VB
    return check_launch();
}

}  // namespace
}  // namespace gsv

using namespace gsv;

extern "C" int gsv_voxelize_fwd(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                                int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                                const int32_t *tile_bins, const float *pos3d_radii,
                                const float *conics, const float *intensities, float *volume,
                                uint8_t *pair_live, void *stream) {
    return voxelize_fwd_impl(D, H, W, channels, n, num_intersects, gaussian_ids_sorted, tile_bins,
                             pos3d_radii, conics, intensities, volume, nullptr, nullptr, nullptr,
                             nullptr, pair_live, as_stream(stream));
}

extern "C" int gsv_voxelize_fwd_l1_workspace_bytes(int32_t D, int32_t H, int32_t W,
                                                   size_t *bytes) {
    if (!bytes || D <= 0 || H <= 0 || W <= 0) return GSV_ERR_INVALID_ARGUMENT;
    const int64_t T = (int64_t)gsv_tiles_along(W) * gsv_tiles_along(H) * gsv_tiles_along(D);
    *bytes = align256((size_t)T * sizeof(float));
    return GSV_OK;
}

extern "C" int gsv_voxelize_fwd_l1(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                                   int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                                   const int32_t *tile_bins, const float *pos3d_radii,
                                   const float *conics, const float *intensities,
                                   const float *target, float *volume, int8_t *sign, float *loss,
                                   uint8_t *pair_live, void *workspace, size_t workspace_bytes,
                                   void *stream) {
    if (!target || !loss || !sign) return GSV_ERR_INVALID_ARGUMENT;
    size_t need = 0;
    if (int st = gsv_voxelize_fwd_l1_workspace_bytes(D, H, W, &need)) return st;
    if (!workspace || workspace_bytes < need) return GSV_ERR_WORKSPACE_TOO_SMALL;
    return voxelize_fwd_impl(D, H, W, channels, n, num_intersects, gaussian_ids_sorted, tile_bins,
                             pos3d_radii, conics, intensities, volume, target,
                             static_cast<float *>(workspace), sign, loss, pair_live,
                             as_stream(stream));
}

extern "C" int gsv_voxelize_bwd_workspace_bytes(int32_t D, int32_t H, int32_t W,
                                                int32_t channels, int32_t n,
                                                int64_t num_intersects, int32_t deterministic,
                                                size_t *bytes) {
    if (!bytes || D <= 0 || H <= 0 || W <= 0 || n < 0) return GSV_ERR_INVALID_ARGUMENT;
    if (channels < 1 || channels > GSV_MAX_CHANNELS) return GSV_ERR_UNSUPPORTED_CHANNELS;
    *bytes = bwd_layout(n, num_intersects > 0 ? num_intersects : 0, channels, deterministic != 0).end;
    return GSV_OK;
}

extern "C" int gsv_voxelize_bwd(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                                int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                                const int32_t *tile_bins, const float *pos3d_radii,
                                const float *conics, const float *intensities,
                                const float *vol_grad, const int32_t *tile_min,
                                const int32_t *tile_max, const int32_t *cum_tiles_hit,
                                const int32_t *tiles_sorted, const int64_t *num_intersects_dev,
                                const uint8_t *pair_live, float *dpos3d_radii, float *dconics,
                                float *dintensities, int32_t variant, void *workspace,
                                size_t workspace_bytes, void *stream) {
    return voxelize_bwd_impl(D, H, W, channels, n, num_intersects, gaussian_ids_sorted, tile_bins,
                             pos3d_radii, conics, intensities, vol_grad, nullptr, nullptr,
                             tile_min, tile_max, cum_tiles_hit, tiles_sorted, num_intersects_dev,
                             pair_live, dpos3d_radii, dconics,
                             dintensities, variant, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int gsv_set_backward_chains(int32_t enabled, int32_t *previous) {
    if (enabled != 0 && enabled != 1) return GSV_ERR_INVALID_ARGUMENT;
    const int before = bwd_chains_enabled() ? 1 : 0;
    g_bwd_chains.store(enabled, std::memory_order_relaxed);
    if (previous) *previous = before;
    return GSV_OK;
}

extern "C" int gsv_voxelize_bwd_l1(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                                   int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                                   const int32_t *tile_bins, const float *pos3d_radii,
                                   const float *conics, const float *intensities,
                                   const int8_t *sign, const float *grad_loss,
                                   const float *vol_grad, const int32_t *tile_min,
                                   const int32_t *tile_max, const int32_t *cum_tiles_hit,
                                   const int32_t *tiles_sorted, const int64_t *num_intersects_dev,
                                   const uint8_t *pair_live, float *dpos3d_radii, float *dconics,
                                   float *dintensities, int32_t variant, void *workspace,
                                   size_t workspace_bytes, void *stream) {
    if (!sign || !grad_loss) return GSV_ERR_INVALID_ARGUMENT;
    return voxelize_bwd_impl(D, H, W, channels, n, num_intersects, gaussian_ids_sorted, tile_bins,
                             pos3d_radii, conics, intensities, vol_grad, sign, grad_loss,
                             tile_min, tile_max, cum_tiles_hit, tiles_sorted, num_intersects_dev,
                             pair_live, dpos3d_radii, dconics,
                             dintensities, variant, workspace, workspace_bytes, as_stream(stream));
}
