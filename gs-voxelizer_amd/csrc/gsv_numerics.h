/*
 * gsv_numerics.h — numerical contract shared, as source, by the gfx950 kernels
 * and by the host C oracle under oracle/.
 *
 * Tile binning (tile_min / tile_max / num_tiles_hit) must match bit for bit
 * between the device and the host.  Everything that feeds the bounding box is
 * therefore written here with IEEE-754 binary32 +, -, *, / and sqrt only, with
 * floating-point contraction switched off (clang: pragma below; gcc: the oracle
 * is built with -ffp-contract=off), and with no call into a vendor math library
 * whose last-bit behaviour differs between libm and the device library.
 *
 * Reference constants: ALPHA_THRESHOLD = 1/1e-6 (gs_voxelizer/cuda/optim_to_render.cuh:7),
 * tile edge 8 (gs_voxelizer/cuda/config.h:1-4), channel limit 4 (config.h:7).
 */
#ifndef GSV_NUMERICS_H
#define GSV_NUMERICS_H

#include <stdint.h>

#if defined(__HIPCC__)
#define GSV_HD __host__ __device__
#else
#define GSV_HD
#endif

#if defined(__clang__)
#define GSV_NO_CONTRACT _Pragma("clang fp contract(off)")
#else
#define GSV_NO_CONTRACT
#endif

#define GSV_TILE 8                 /* voxels per tile edge (config.h:1-3)          */
#define GSV_TILE_VOXELS 512        /* GSV_TILE^3                                    */
#define GSV_MAX_CHANNELS 4         /* config.h:7                                    */
#define GSV_ALPHA_THRESHOLD 1000000.0f /* 1/0.000001f rounded to binary32 = 1e6 exactly */
#define GSV_MIN_CONTRIB 0.000001f  /* per-voxel contribution gate (voxelize.cu:146)  */

static inline GSV_HD uint32_t gsv_f2u(float x) {
    uint32_t u;
    __builtin_memcpy(&u, &x, sizeof u);
    return u;
}

static inline GSV_HD float gsv_u2f(uint32_t u) {
    float x;
    __builtin_memcpy(&x, &u, sizeof x);
    return x;
}

/*
 * Natural logarithm in binary32.
 *
 * Method (Cody & Waite range reduction; series from the identity
 * log(m) = 2 atanh((m-1)/(m+1))):
 *   x = 2^k * m with m in [sqrt(1/2), sqrt(2)),
 *   s = (m-1)/(m+1), |s| <= 0.1716, z = s*s <= 0.0295,
 *   log(m) = 2s * (1 + z/3 + z^2/5 + ... + z^6/13)   (next term < 2e-12 relative),
 *   log(x) = k*ln2_hi + (log(m) + k*ln2_lo),
 * with ln2_hi = 0x3f317000 (12 trailing zero bits, so k*ln2_hi is exact for
 * |k| < 2^12) and ln2_lo = binary32(ln2 - ln2_hi).  Special values follow C99:
 * log(+0) = -inf, log(x<0) = NaN, log(NaN) = NaN, log(+inf) = +inf.
 * Accuracy is a few ulp; what matters here is that host and device agree exactly.
 */
static inline GSV_HD float gsv_logf(float x) {
    GSV_NO_CONTRACT
    if (!(x > 0.0f)) {
        if (x == 0.0f) return -gsv_u2f(0x7f800000u);
        return gsv_u2f(0x7fc00000u);
    }
    uint32_t ix = gsv_f2u(x);
    if (ix >= 0x7f800000u) return x;               /* +inf */
    int k = 0;
    if (ix < 0x00800000u) {                        /* subnormal: scale by 2^23 */
        x = x * 8388608.0f;
        ix = gsv_f2u(x);
        k = -23;
    }
    k += (int)(ix >> 23) - 127;
    float m = gsv_u2f((ix & 0x007fffffu) | 0x3f800000u); /* m in [1, 2) */
    if (m > 1.41421354f) {
        m = m * 0.5f;
        k += 1;
    }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    float p = 0.0769230798f;          /* 1/13 */
    p = p * z + 0.0909090936f;        /* 1/11 */
    p = p * z + 0.111111112f;         /* 1/9  */
    p = p * z + 0.142857149f;         /* 1/7  */
    p = p * z + 0.200000003f;         /* 1/5  */
    p = p * z + 0.333333343f;         /* 1/3  */
    p = p * z;
    const float two_s = s + s;
    const float log_m = two_s + two_s * p;
    const float kf = (float)k;
    return kf * 0.693115234f + (log_m + kf * 3.19461833e-05f);
}

/*
 * Float -> int32 conversion with round-toward-zero and saturation, NaN -> 0.
 * This is the semantics of the device conversion the reference's `(int)` casts
 * compile to (get_tile_bbox, optim_to_render.cu:26-40); plain C leaves the
 * out-of-range case undefined, so the host spells it out.
 */
static inline GSV_HD int gsv_f2i_sat(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return 2147483647;
    if (v <= -2147483648.0f) return (-2147483647 - 1);
    return (int)v;
}

static inline GSV_HD int gsv_imin(int a, int b) { return a < b ? a : b; }
static inline GSV_HD int gsv_imax(int a, int b) { return a > b ? a : b; }

/* Tile grid for a (D, H, W) volume: (ceil(W/8), ceil(H/8), ceil(D/8)) — bindings.cu:70-74. */
static inline GSV_HD int gsv_tiles_along(int n) { return (n + GSV_TILE - 1) / GSV_TILE; }

#endif /* GSV_NUMERICS_H */
