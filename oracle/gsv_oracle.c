/*
 * gsv_oracle.c — CPU restatement of the reference voxelization path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the gfx950 kernels are
 * compared against; it is never linked into, loaded by, or called from the
 * product path (gs-voxelizer_amd/).  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it.
 *
 * Build: oracle/build_oracle.sh (gcc -O2 -std=c11 -ffp-contract=off -fopenmp).
 * Every arithmetic expression keeps the reference's evaluation order in
 * binary32 with no contraction, so that the integer bin outputs are defined
 * by IEEE-754 and can be compared bit for bit with the device.  The same
 * source built with -DORC_BINARY64 is the binary64 twin described below.
 *
 * Reference = PaPieta/gs-voxelizer v0.1.0; citations are path:line under
 * gs_voxelizer/.  GLM mat3 semantics are restated explicitly: matrices are
 * column-major, m[c][r] is column c row r, and (A*B)[c][r] =
 * A[0][r]*B[c][0] + A[1][r]*B[c][1] + A[2][r]*B[c][2] summed left to right.
 *
 * Parity status of each entry point is documented next to it ("pinned by").
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <tgmath.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../gs-voxelizer_amd/csrc/gsv_numerics.h"

/*
 * Arithmetic type.  The default build (liboracle.so) computes in binary32, the
 * reference's type, in its evaluation order.  -DORC_BINARY64 builds the same
 * source in binary64 (liboracle64.so): the same formulas, operation for
 * operation, with the reference's binary32 constants (1e-7f, 1e-6f) kept as
 * they are, and the natural log from libm.  Fed binary32 inputs, it estimates
 * the exact value of each output to ~1e-16 relative, which is what the tests
 * measure the binary32 evaluations (this oracle's and the device's) against.
 * Math calls go through <tgmath.h>, so each resolves to the type's function.
 */
#ifdef ORC_BINARY64
typedef double real;
#define orc_log(x) log(x)
#else
typedef float real;
#define orc_log(x) gsv_logf(x)
#endif

typedef real mat3[3][3]; /* [col][row], GLM layout */

static void m3_mul(mat3 out, mat3 a, mat3 b) {
    mat3 r;
    for (int c = 0; c < 3; ++c)
        for (int row = 0; row < 3; ++row)
            r[c][row] = a[0][row] * b[c][0] + a[1][row] * b[c][1] + a[2][row] * b[c][2];
    memcpy(out, r, sizeof(mat3));
}

static void m3_transpose(mat3 out, mat3 a) {
    mat3 r;
    for (int c = 0; c < 3; ++c)
        for (int row = 0; row < 3; ++row) r[c][row] = a[row][c];
    memcpy(out, r, sizeof(mat3));
}

/* glm::mat3(a0..a8): column-major constructor. */
static void m3_set(mat3 m, real a0, real a1, real a2, real a3, real a4, real a5,
                   real a6, real a7, real a8) {
    m[0][0] = a0; m[0][1] = a1; m[0][2] = a2;
    m[1][0] = a3; m[1][1] = a4; m[1][2] = a5;
    m[2][0] = a6; m[2][1] = a7; m[2][2] = a8;
}

/* quaternion [w,x,y,z] -> rotation, optim_to_render_helpers.cuh:15-36.
 * The reference normalises with rsqrtf; the restatement uses 1/sqrtf. The
 * squared norm is summed in the order the reference reads the float4
 * (.w,.x,.y,.z = q3,q0,q1,q2). */
static void quat_to_rotmat(const real *q, mat3 R, real *wxyz) {
    const real n2 = q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2];
    const real s = 1.0f / sqrt(n2);
    const real w = q[0] * s, x = q[1] * s, y = q[2] * s, z = q[3] * s;
    m3_set(R,
           1.f - 2.f * (y * y + z * z), 2.f * (x * y - w * z), 2.f * (x * z + w * y),
           2.f * (x * y + w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z - w * x),
           2.f * (x * z - w * y), 2.f * (y * z + w * x), 1.f - 2.f * (x * x + y * y));
    if (wxyz) { wxyz[0] = w; wxyz[1] = x; wxyz[2] = y; wxyz[3] = z; }
}

/* Voxel-space covariance, optim_to_render.cu:85-103 (forward) and 280-300 (backward).
 * vs3 = (vs.x, vs.y, vs.z) in the kernel's dim3 order (D,H,W), i.e. (z,y,x) sizes. */
static void voxel_covariance(const real *scale, const real *quat, const real vs3[3],
                             mat3 R, mat3 S, mat3 M2, mat3 cov) {
    m3_set(S, 1.f, 0.f, 0.f, 0.f, 1.f, 0.f, 0.f, 0.f, 1.f);
    S[0][0] = scale[0];
    S[1][1] = scale[1];
    S[2][2] = scale[2];
    quat_to_rotmat(quat, R, NULL);
    mat3 M, Mt;
    m3_mul(M, S, R);
    m3_transpose(Mt, M);
    m3_mul(cov, Mt, M);
    m3_set(M2, 1.f / vs3[2], 0.0f, 0.0f, 0.0f, 1.f / vs3[1], 0.0f, 0.0f, 0.0f, 1.f / vs3[0]);
    mat3 M2t;
    m3_transpose(M2t, M2);
    m3_mul(cov, M2t, cov);
    m3_mul(cov, cov, M2);
}

/*
 * Projection forward: optim_to_render.cu:48-172 (+ get_tile_bbox 26-40),
 * driven as bindings.cu:59-96 does (outputs zeroed first; (D,H,W) in dim3 order).
 * Pinned by: tests/test_oracle_projection.py (closed forms, fp64 linear algebra,
 * hand-computed boxes, special values).
 */
int orc_project_fwd(int n, int C, const real *pos3d, const real *scale3d, const real *quat,
                     const real *intens, int D, int H, int W, real wz, real wy, real wx,
                     real cz, real cy, real cx, real *pos_radii, real *conics, int *tile_min,
                     int *tile_max, int *num_tiles_hit) {
    if (n < 0 || C < 1 || C > GSV_MAX_CHANNELS) return 1;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    const real vs3[3] = {wz / (real)D, wy / (real)H, wx / (real)W};
    memset(pos_radii, 0, sizeof(real) * 4 * (size_t)n);
    memset(conics, 0, sizeof(real) * 6 * (size_t)n);
    memset(tile_min, 0, sizeof(int) * 3 * (size_t)n);
    memset(tile_max, 0, sizeof(int) * 3 * (size_t)n);
    memset(num_tiles_hit, 0, sizeof(int) * (size_t)n);
#pragma omp parallel for schedule(static)
    for (int g = 0; g < n; ++g) {
        const real *p = pos3d + 3 * (size_t)g, *s = scale3d + 3 * (size_t)g;
        const real pix[3] = {(p[0] - cx + (wx * 0.5f)) / vs3[2],
                              (p[1] - cy + (wy * 0.5f)) / vs3[1],
                              (p[2] - cz + (wz * 0.5f)) / vs3[0]};
        mat3 R, S, M2, cov;
        voxel_covariance(s, quat + 4 * (size_t)g, vs3, R, S, M2, cov);
        const real a = cov[0][0], b = cov[0][1], c = cov[0][2];
        const real d = cov[1][1], e = cov[1][2], f = cov[2][2];
        const real det = a * d * f + 2 * b * c * e - a * e * e - f * b * b - d * c * c;
        if (det == 0.0f) continue;
        const real inv_det = 1.0f / det;
        const real ia = inv_det * (d * f - e * e);
        const real ib = inv_det * (c * e - b * f);
        const real ic = inv_det * (b * e - c * d);
        const real id = inv_det * (a * f - c * c);
        const real ie = inv_det * (b * c - a * e);
        const real iff = inv_det * (a * d - b * b);
        const real radius = ceil((3.f * fmax(s[0], fmax(s[1], s[2]))) /
                                   fmin(vs3[2], fmin(vs3[1], vs3[0])));
        real mean = 0.f;
        for (int ch = 0; ch < C; ++ch) mean += intens[(size_t)g * C + ch];
        mean /= (real)C;
        const real opt = orc_log(mean * GSV_ALPHA_THRESHOLD);
        const real extent = fmin(3.f, sqrt(2.0f * opt));
        const real r3[3] = {fmax(0.0f, (sqrt(cov[0][0]) * extent) - 0.5f),
                             fmax(0.0f, (sqrt(cov[1][1]) * extent) - 0.5f),
                             fmax(0.0f, (sqrt(cov[2][2]) * extent) - 0.5f)};
        if (radius <= 0.f || pix[0] + radius < 0.f || pix[0] - radius > (real)W ||
            pix[1] + radius < 0.f || pix[1] - radius > (real)H || pix[2] + radius < 0.f ||
            pix[2] - radius > (real)D)
            continue;
        const int tb[3] = {Tx, Ty, Tz};
        int tmn[3], tmx[3];
        for (int k = 0; k < 3; ++k) {
            tmn[k] = gsv_imin(tb[k], gsv_imax(0, gsv_f2i_sat((pix[k] - r3[k]) / (real)GSV_TILE)));
            tmx[k] = gsv_imin(tb[k], gsv_imax(0, gsv_f2i_sat((pix[k] + r3[k] + (real)(GSV_TILE - 1)) /
                                                              (real)GSV_TILE)));
        }
        const int tile_vol = (tmx[0] - tmn[0]) * (tmx[1] - tmn[1]) * (tmx[2] - tmn[2]);
        if (tile_vol <= 0) continue;
        real *pr = pos_radii + 4 * (size_t)g;
        pr[0] = pix[0]; pr[1] = pix[1]; pr[2] = pix[2]; pr[3] = radius;
        for (int k = 0; k < 3; ++k) {
            tile_min[3 * (size_t)g + k] = tmn[k];
            tile_max[3 * (size_t)g + k] = tmx[k];
        }
        num_tiles_hit[g] = tile_vol;
        real *cn = conics + 6 * (size_t)g;
        cn[0] = ia; cn[1] = ib; cn[2] = ic; cn[3] = id; cn[4] = ie; cn[5] = iff;
    }
    return 0;
}

/* dL/d(voxel covariance) from dL/d(conic), get_cov_grad optim_to_render.cu:186-239. */
static void cov_grad_from_conic_grad(mat3 cov, mat3 M2, const real *g, mat3 out) {
    const real a = cov[0][0], b = cov[0][1], c = cov[0][2];
    const real d = cov[1][1], e = cov[1][2], f = cov[2][2];
    const real den = a * d * f + 2 * b * c * e - a * e * e - f * b * b - d * c * c;
    const real den2inv = 1.0f / ((den * den) + 0.0000001f);
    m3_set(out, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f);
    if (den2inv == 0) return;
    /* cofactors and det partials */
    const real k_a = d * f - e * e;
    const real k_b = 2 * c * e - 2 * f * b;
    const real k_c = 2 * b * e - 2 * d * c;
    const real k_d = a * f - c * c;
    const real k_e = 2 * b * c - 2 * a * e;
    const real k_f = a * d - b * b;
    const real n_b = c * e - b * f;
    const real n_c = b * e - c * d;
    const real n_e = b * c - a * e;
    const real gA = g[0], gB = g[1], gC = g[2], gD = g[3], gE = g[4], gF = g[5];
    const real da = den2inv * (-k_a * k_a * gA - n_b * k_a * gB - n_c * k_a * gC +
                                (f * den - k_d * k_a) * gD + (-e * den - n_e * k_a) * gE +
                                (d * den - k_f * k_a) * gF);
    const real db = den2inv * (-k_a * k_b * gA + (-f * den - n_b * k_b) * gB +
                                (e * den - n_c * k_b) * gC - k_d * k_b * gD +
                                (c * den - n_e * k_b) * gE + (-2 * b * den - k_f * k_b) * gF);
    const real dc = den2inv * (-k_a * k_c * gA + (e * den - n_b * k_c) * gB +
                                (-d * den - n_c * k_c) * gC + (-2 * c * den - k_d * k_c) * gD +
                                (b * den - n_e * k_c) * gE - k_f * k_c * gF);
    const real dd = den2inv * ((f * den - k_a * k_d) * gA - n_b * k_d * gB +
                                (-c * den - n_c * k_d) * gC - k_d * k_d * gD - n_e * k_d * gE +
                                (a * den - k_f * k_d) * gF);
    const real de = den2inv * ((-2 * e * den - k_a * k_e) * gA + (c * den - n_b * k_e) * gB +
                                (b * den - n_c * k_e) * gC - k_d * k_e * gD +
                                (-a * den - n_e * k_e) * gE + -k_f * k_e * gF);
    const real df = den2inv * ((d * den - k_a * k_f) * gA + (-b * den - n_b * k_f) * gB -
                                n_c * k_f * gC + (a * den - k_d * k_f) * gD - n_e * k_f * gE -
                                k_f * k_f * gF);
    mat3 dhat, M2t, t;
    m3_set(dhat, da, db, dc, db, dd, de, dc, de, df);
    m3_transpose(M2t, M2);
    m3_mul(t, M2, dhat);
    m3_mul(t, t, M2t);
    for (int col = 0; col < 3; ++col)
        for (int row = 0; row < 3; ++row) out[col][row] = 0.5f * (t[col][row] + t[row][col]);
}

/*
 * Projection backward: optim_to_render.cu:246-336 with helpers 51-75,
 * driven as bindings.cu:213-243 (outputs zeroed first).
 * Pinned by: tests/test_oracle_projection.py (fp64 finite differences on dscale,
 * tangential dquat, dpos up to the reference's voxel-size factor).
 */
int orc_project_bwd(int n, const real *pos3d, const real *scale3d, const real *quat, int D,
                    int H, int W, real wz, real wy, real wx, real cz, real cy, real cx,
                    const real *dpos_radii, const real *dconics, const real *pos_radii,
                    real *dpos, real *dscale, real *dquat) {
    (void)pos3d; (void)cz; (void)cy; (void)cx;
    if (n < 0) return 1;
    const real vs3[3] = {wz / (real)D, wy / (real)H, wx / (real)W};
    memset(dpos, 0, sizeof(real) * 3 * (size_t)n);
    memset(dscale, 0, sizeof(real) * 3 * (size_t)n);
    memset(dquat, 0, sizeof(real) * 4 * (size_t)n);
#pragma omp parallel for schedule(static)
    for (int g = 0; g < n; ++g) {
        if (pos_radii[4 * (size_t)g + 3] <= 0) continue;
        const real *s = scale3d + 3 * (size_t)g;
        const real *q = quat + 4 * (size_t)g;
        mat3 R, S, M2, cov, cg, dsig, Rg, Rgt, Rt, S2;
        voxel_covariance(s, q, vs3, R, S, M2, cov);
        cov_grad_from_conic_grad(cov, M2, dconics + 6 * (size_t)g, cg);
        m3_set(dsig, cg[0][0], 0.5f * cg[0][1], 0.5f * cg[0][2], 0.5f * cg[1][0], cg[1][1],
               0.5f * cg[1][2], 0.5f * cg[2][0], 0.5f * cg[2][1], cg[2][2]);
        for (int col = 0; col < 3; ++col)
            for (int row = 0; row < 3; ++row) S2[col][row] = 2.0f * S[col][row];
        m3_mul(Rg, S2, R);
        m3_mul(Rg, Rg, dsig);
        m3_transpose(Rgt, Rg);
        m3_transpose(Rt, R);
        for (int i = 0; i < 3; ++i)
            dscale[3 * (size_t)g + i] = Rt[i][0] * Rgt[i][0] + Rt[i][1] * Rgt[i][1] + Rt[i][2] * Rgt[i][2];
        for (int i = 0; i < 3; ++i)
            for (int row = 0; row < 3; ++row) Rgt[i][row] *= s[i];
        const real *dp = dpos_radii + 4 * (size_t)g;
        dpos[3 * (size_t)g + 0] = dp[0] * vs3[2];
        dpos[3 * (size_t)g + 1] = dp[1] * vs3[1];
        dpos[3 * (size_t)g + 2] = dp[2] * vs3[0];
        /* rotmat_grad_to_quat_grad, optim_to_render_helpers.cuh:51-75 */
        real qn[4];
        mat3 Rdummy;
        quat_to_rotmat(q, Rdummy, qn);
        const real w = qn[0], x = qn[1], y = qn[2], z = qn[3];
        real (*v)[3] = Rgt;
        real *o = dquat + 4 * (size_t)g;
        o[0] = 2 * z * (v[0][1] - v[1][0]) + 2 * y * (v[2][0] - v[0][2]) + 2 * x * (v[1][2] - v[2][1]);
        o[1] = 2 * y * (v[1][0] + v[0][1]) + 2 * z * (v[2][0] + v[0][2]) + 2 * w * (v[1][2] - v[2][1]) -
               4 * x * (v[2][2] + v[1][1]);
        o[2] = 2 * x * (v[1][0] + v[0][1]) + 2 * w * (v[2][0] - v[0][2]) + 2 * z * (v[1][2] + v[2][1]) -
               4 * y * (v[2][2] + v[0][0]);
        o[3] = 2 * w * (v[0][1] - v[1][0]) + 2 * x * (v[2][0] + v[0][2]) + 2 * y * (v[1][2] + v[2][1]) -
               4 * z * (v[1][1] + v[0][0]);
    }
    return 0;
}

/* Inclusive prefix sum of num_tiles_hit in int32 (torch.cumsum, voxelize.py:87). */
void orc_cumsum_i32(int n, const int *x, int *out) {
    int acc = 0;
    for (int i = 0; i < n; ++i) {
        acc += x[i];
        out[i] = acc;
    }
}

/*
 * Binning: map_gaussian_to_intersects (bin_and_sort_gaussians.cu:11-35) emits
 * (tile_id, g) gaussian-major with tiles in z->y->x nested order; the stable
 * 32-bit radix sort (bindings.cu:313-345) then orders by tile, keeping emission
 * order within a tile; get_tile_bin_edges (bin_and_sort_gaussians.cu:40-62)
 * records [start, end) per non-empty tile, empty tiles stay (0, 0).
 * Restated as a stable counting sort, which produces the identical sequence.
 * Pinned by: tests/test_oracle_binning.py (Python sorted() brute force).
 * keys_sorted may be NULL.  Returns 0, or 2 if cum[-1] != n_isect.
 */
int orc_bin_and_sort(int n, int64_t n_isect, const int *tile_min, const int *tile_max,
                     const int *cum, int D, int H, int W, int *ids_sorted, int *tile_bins,
                     int *keys_sorted) {
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    const int64_t T = (int64_t)Tx * Ty * Tz;
    memset(tile_bins, 0, sizeof(int) * 2 * (size_t)T);
    if (n_isect <= 0) return 0;
    if (n > 0 && (int64_t)cum[n - 1] != n_isect) return 2;
    int64_t *count = (int64_t *)calloc((size_t)T + 1, sizeof(int64_t));
    for (int g = 0; g < n; ++g) {
        const int *mn = tile_min + 3 * (size_t)g, *mx = tile_max + 3 * (size_t)g;
        for (int i = mn[2]; i < mx[2]; ++i)
            for (int j = mn[1]; j < mx[1]; ++j)
                for (int k = mn[0]; k < mx[0]; ++k) count[(int64_t)i * Ty * Tx + (int64_t)j * Tx + k]++;
    }
    int64_t run = 0;
    for (int64_t t = 0; t < T; ++t) {
        const int64_t c = count[t];
        if (c > 0) {
            tile_bins[2 * t] = (int)run;
            tile_bins[2 * t + 1] = (int)(run + c);
        }
        count[t] = run;
        run += c;
    }
    for (int g = 0; g < n; ++g) {
        const int *mn = tile_min + 3 * (size_t)g, *mx = tile_max + 3 * (size_t)g;
        for (int i = mn[2]; i < mx[2]; ++i)
            for (int j = mn[1]; j < mx[1]; ++j)
                for (int k = mn[0]; k < mx[0]; ++k) {
                    const int64_t t = (int64_t)i * Ty * Tx + (int64_t)j * Tx + k;
                    const int64_t slot = count[t]++;
                    ids_sorted[slot] = g;
                    if (keys_sorted) keys_sorted[slot] = (int)t;
                }
    }
    free(count);
    return 0;
}

/*
 * True when an evaluation sits so close to one of the two gates that binary32
 * rounding decides whether it counts: alpha*mean within 1e-4 (relative) of the
 * 1e-6 threshold, or |sigma| < 1e-5 around the sigma <= 0 gate.  Any two fp32
 * evaluation orders (this oracle, the device, the reference's fast-math build)
 * can disagree on such terms; the tests allow their magnitude explicitly.
 */
static int gate_ambiguous(real sigma, real mean, real alpha) {
    if (isnan(sigma) || isinf(sigma) || !(mean > 0.f)) return 0;
    if (fabs(sigma) < 1e-5f) return 1;
    if (sigma > 0.f) return 0;
    /* alpha = exp(sigma) in the working type (a few ulp): far from the band
     * when alpha*mean is off 1e-6 by more than twice its width */
    if (fabs((double)alpha * (double)mean - 1e-6) > 2e-10) return 0;
    const double am = exp((double)sigma) * (double)mean;
    return fabs(am - 1e-6) <= 1e-4 * 1e-6;
}

/*
 * Forward voxelization: voxelize_forward (voxelize.cu:39-164).  Each inside
 * voxel sums, in ascending position within its tile's list, I_c * exp(sigma)
 * over Gaussians that pass both gates.  Tiles [tile_begin, tile_end) only;
 * voxels of other tiles are left untouched (the caller zero-fills).
 * amb (optional, same layout as out) receives per voxel the sum of |I_c*alpha|
 * over gate-ambiguous evaluations (see gate_ambiguous).
 * out and amb hold the z planes [z_base, z_base + z_count) of the volume
 * (z_base = 0, z_count = D for the whole volume); voxels of other planes are
 * skipped.
 * Pinned by: tests/test_oracle_voxelize.py (dense fp64 brute force, closed forms).
 */
int orc_voxelize_fwd(int D, int H, int W, int C, const int *ids_sorted, const int *tile_bins,
                     const real *pos_radii, const real *conics, const real *intens, real *out,
                     real *amb, int64_t tile_begin, int64_t tile_end, int z_base, int z_count) {
    if (C < 1 || C > GSV_MAX_CHANNELS) return 1;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H);
    const int64_t T = (int64_t)Tx * Ty * gsv_tiles_along(D);
    if (tile_end > T) tile_end = T;
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t t = tile_begin; t < tile_end; ++t) {
        const int tx = (int)(t % Tx), ty = (int)((t / Tx) % Ty), tz = (int)(t / ((int64_t)Tx * Ty));
        const int r0 = tile_bins[2 * t], r1 = tile_bins[2 * t + 1];
        for (int lz = 0; lz < GSV_TILE; ++lz)
            for (int ly = 0; ly < GSV_TILE; ++ly)
                for (int lx = 0; lx < GSV_TILE; ++lx) {
                    const int i = tz * GSV_TILE + lz, j = ty * GSV_TILE + ly, k = tx * GSV_TILE + lx;
                    if (i >= D || j >= H || k >= W) continue;
                    if (i < z_base || i >= z_base + z_count) continue;
                    const real px = (real)k + 0.5f, py = (real)j + 0.5f, pz = (real)i + 0.5f;
                    real acc[GSV_MAX_CHANNELS] = {0.f, 0.f, 0.f, 0.f};
                    real am[GSV_MAX_CHANNELS] = {0.f, 0.f, 0.f, 0.f};
                    for (int idx = r0; idx < r1; ++idx) {
                        const int g = ids_sorted[idx];
                        const real *xyz = pos_radii + 4 * (size_t)g;
                        const real *cn = conics + 6 * (size_t)g;
                        const real dx = xyz[0] - px, dy = xyz[1] - py, dz = xyz[2] - pz;
                        const real sigma = -0.5f * (cn[0] * dx * dx + cn[3] * dy * dy + cn[5] * dz * dz) -
                                            (cn[1] * dx * dy + cn[2] * dx * dz + cn[4] * dy * dz);
                        real mean = 0.f;
                        for (int ch = 0; ch < C; ++ch) mean += intens[(size_t)g * C + ch];
                        mean /= (real)C;
                        /* exp(sigma) wherever sigma <= 0 (the only case used below) */
                        const real alpha = exp(fmin(sigma, 0.f));
                        if (amb && gate_ambiguous(sigma, mean, alpha))
                            for (int ch = 0; ch < C; ++ch)
                                am[ch] += fabs(intens[(size_t)g * C + ch] * alpha);
                        if (sigma > 0.f || isnan(sigma) || isinf(sigma)) continue;
                        if (alpha * mean < GSV_MIN_CONTRIB) continue;
                        for (int ch = 0; ch < C; ++ch) acc[ch] += intens[(size_t)g * C + ch] * alpha;
                    }
                    const size_t at = ((((size_t)(i - z_base) * H + j) * W) + k) * C;
                    for (int ch = 0; ch < C; ++ch) out[at + ch] = acc[ch];
                    if (amb)
                        for (int ch = 0; ch < C; ++ch) amb[at + ch] = am[ch];
                }
    }
    return 0;
}

/*
 * Backward voxelization: voxelize_backward_per_gaussian (voxelize.cu:368-574).
 * For each (tile, Gaussian) pair the per-voxel terms are summed in the
 * arithmetic type (binary32 by default) in the kernel's voxel order (z, then y, then x within the tile), as one lane of
 * the reference does; the per-pair partials are then added into each
 * Gaussian's gradient in binary64, in sorted pair order (the reference uses
 * float atomics in an unspecified order).  Outputs are zeroed first
 * (bindings.cu:630-632); dpos_radii[:,3] stays 0.
 *
 * Optional diagnostics, same layouts as the gradients (pass NULL to skip):
 *   abs_*: per element, the sum of |term| over every contributing voxel — the
 *          conditioning of the sum, which bounds summation-order error;
 *   amb_*: per element, the sum of |term| over gate-ambiguous evaluations
 *          (gate_ambiguous), whether or not this oracle counted them.
 * Pairs of tiles outside [tile_begin, tile_end) are skipped.
 * Pinned by: tests/test_oracle_voxelize.py (torch autograd of a dense fp64
 * evaluation of the forward, and central finite differences).
 */
static void bwd_terms(real sg, real dd, const real *vg, int C, real dx, real dy, real dz,
                      const real *cn, real *term) {
    for (int ch = 0; ch < C; ++ch) term[9 + ch] = dd * vg[ch];
    term[0] = -0.5f * sg * dx * dx;
    term[1] = -sg * dx * dy;
    term[2] = -sg * dx * dz;
    term[3] = -0.5f * sg * dy * dy;
    term[4] = -sg * dy * dz;
    term[5] = -0.5f * sg * dz * dz;
    term[6] = -sg * (cn[0] * dx + cn[1] * dy + cn[2] * dz);
    term[7] = -sg * (cn[1] * dx + cn[3] * dy + cn[4] * dz);
    term[8] = -sg * (cn[2] * dx + cn[4] * dy + cn[5] * dz);
}

int orc_voxelize_bwd(int D, int H, int W, int C, int n, const int *ids_sorted, const int *tile_bins,
                     const real *pos_radii, const real *conics, const real *intens,
                     const real *vol_grad, real *dpos_radii, real *dconics, real *dintens,
                     real *abs_pos, real *abs_conics, real *abs_intens, real *amb_pos,
                     real *amb_conics, real *amb_intens, int64_t tile_begin, int64_t tile_end) {
    if (C < 1 || C > GSV_MAX_CHANNELS) return 1;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H);
    const int64_t T = (int64_t)Tx * Ty * gsv_tiles_along(D);
    if (tile_end > T) tile_end = T;
    const int NV = 9 + C;
    const int want_abs = abs_pos != NULL, want_amb = amb_pos != NULL;
    memset(dpos_radii, 0, sizeof(real) * 4 * (size_t)n);
    memset(dconics, 0, sizeof(real) * 6 * (size_t)n);
    memset(dintens, 0, sizeof(real) * (size_t)C * n);
    real *outs[3][3] = {{dconics, dpos_radii, dintens}, {abs_conics, abs_pos, abs_intens},
                         {amb_conics, amb_pos, amb_intens}};
    for (int k = 1; k < 3; ++k)
        if (outs[k][0]) {
            memset(outs[k][0], 0, sizeof(real) * 6 * (size_t)n);
            memset(outs[k][1], 0, sizeof(real) * 4 * (size_t)n);
            memset(outs[k][2], 0, sizeof(real) * (size_t)C * n);
        }
    if (tile_begin >= tile_end) return 0;
    /* pairs are sorted by tile, so the pairs of a tile range are contiguous */
    int64_t p0 = INT64_MAX, p1 = 0;
    for (int64_t t = tile_begin; t < tile_end; ++t) {
        if (tile_bins[2 * t + 1] <= tile_bins[2 * t]) continue;
        if (tile_bins[2 * t] < p0) p0 = tile_bins[2 * t];
        if (tile_bins[2 * t + 1] > p1) p1 = tile_bins[2 * t + 1];
    }
    if (p1 <= p0) return 0;
    const int64_t npairs = p1 - p0;
    /* per pair: the partial sums, then (with diagnostics) |term| and ambiguous sums */
    const int K = (want_abs || want_amb) ? 3 : 1;
    real *part = (real *)calloc((size_t)npairs * NV * K, sizeof(real));
    if (!part) return 3;
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t t = tile_begin; t < tile_end; ++t) {
        const int tx = (int)(t % Tx), ty = (int)((t / Tx) % Ty), tz = (int)(t / ((int64_t)Tx * Ty));
        const int r0 = tile_bins[2 * t], r1 = tile_bins[2 * t + 1];
        for (int idx = r0; idx < r1; ++idx) {
            const int g = ids_sorted[idx];
            const real *xyz = pos_radii + 4 * (size_t)g;
            const real *cn = conics + 6 * (size_t)g;
            const real *Ig = intens + (size_t)g * C;
            real mean = 0.f;
            for (int ch = 0; ch < C; ++ch) mean += Ig[ch];
            mean /= (real)C;
            real acc[13] = {0}, aac[13] = {0}, amb[13] = {0}, term[13];
            for (int v = 0; v < GSV_TILE_VOXELS; ++v) {
                const int lz = v / 64, ly = (v / 8) % 8, lx = v % 8;
                const int gx = tx * GSV_TILE + lx, gy = ty * GSV_TILE + ly, gz = tz * GSV_TILE + lz;
                if (gx >= W || gy >= H || gz >= D) continue;
                const real px = (real)gx + 0.5f, py = (real)gy + 0.5f, pz = (real)gz + 0.5f;
                const real *vg = vol_grad + ((((size_t)gz * H + gy) * W) + gx) * C;
                const real dx = xyz[0] - px, dy = xyz[1] - py, dz = xyz[2] - pz;
                const real sigma = -0.5f * (cn[0] * dx * dx + cn[3] * dy * dy + cn[5] * dz * dz) -
                                    (cn[1] * dx * dy + cn[2] * dx * dz + cn[4] * dy * dz);
                /* exp(sigma) wherever sigma <= 0 (the only case used below) */
                const real dd = exp(fmin(sigma, 0.f));
                if (want_amb && gate_ambiguous(sigma, mean, dd)) {
                    real sa = 0.f;
                    for (int ch = 0; ch < C; ++ch) sa += Ig[ch] * vg[ch];
                    bwd_terms(sa * dd, dd, vg, C, dx, dy, dz, cn, term);
                    for (int q = 0; q < NV; ++q) amb[q] += fabs(term[q]);
                }
                if (sigma > 0.f || isnan(sigma) || isinf(sigma)) continue;
                if (dd * mean < GSV_MIN_CONTRIB) continue;
                real sg = 0.f;
                for (int ch = 0; ch < C; ++ch) sg += Ig[ch] * vg[ch];
                sg *= dd;
                bwd_terms(sg, dd, vg, C, dx, dy, dz, cn, term);
                for (int q = 0; q < NV; ++q) {
                    acc[q] += term[q];
                    aac[q] += fabs(term[q]);
                }
            }
            real *dst = part + (size_t)(idx - p0) * NV * K;
            for (int q = 0; q < NV; ++q) {
                dst[q] = acc[q];
                if (K == 3) {
                    dst[NV + q] = aac[q];
                    dst[2 * NV + q] = amb[q];
                }
            }
        }
    }
    double *gacc = (double *)calloc((size_t)n * NV * 3 + 1, sizeof(double));
    if (!gacc) { free(part); return 3; }
    for (int64_t t = tile_begin; t < tile_end; ++t) {
        const int r0 = tile_bins[2 * t], r1 = tile_bins[2 * t + 1];
        for (int idx = r0; idx < r1; ++idx) {
            const int g = ids_sorted[idx];
            const real *src = part + (size_t)(idx - p0) * NV * K;
            double *dst = gacc + (size_t)g * NV * 3;
            for (int q = 0; q < K * NV; ++q) dst[q] += (double)src[q];
        }
    }
    for (int g = 0; g < n; ++g) {
        for (int k = 0; k < 3; ++k) {
            if (k == 1 && !want_abs) continue;
            if (k == 2 && !want_amb) continue;
            const double *a = gacc + (size_t)g * NV * 3 + (size_t)k * NV;
            for (int q = 0; q < 6; ++q) outs[k][0][6 * (size_t)g + q] = (real)a[q];
            for (int q = 0; q < 3; ++q) outs[k][1][4 * (size_t)g + q] = (real)a[6 + q];
            for (int ch = 0; ch < C; ++ch) outs[k][2][(size_t)g * C + ch] = (real)a[9 + ch];
        }
    }
    free(gacc);
    free(part);
    return 0;
}

/* Exposed for the log accuracy test. */
float orc_logf(float x) { return gsv_logf(x); }
int orc_f2i_sat(float x) { return gsv_f2i_sat(x); }

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
