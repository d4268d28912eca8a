// project.hip — projection forward/backward for gfx950.
//
// One lane per Gaussian.  The arithmetic follows the reference's evaluation
// order (GLM column-major mat3 products summed left to right) in binary32 with
// contraction off, so that the tile box — and therefore binning — is defined
// by IEEE-754 and reproducible on the host (see gsv_numerics.h).  Reference:
// gs_voxelizer/cuda/optim_to_render.cu:26-172 (forward), 186-336 (backward),
// optim_to_render_helpers.cuh:15-75, launch conventions bindings.cu:38-251.
//
// Culled Gaussians are written as zero rows by the kernel itself, which
// replaces the reference's five memsets (bindings.cu:92-96) with no extra pass.
#include "gsv_device.h"

namespace gsv {
namespace {

// GLM-layout 3x3: m[c][r] = column c, row r.
struct M3 {
    float m[3][3];
};

__device__ __forceinline__ M3 m3(float a0, float a1, float a2, float a3, float a4, float a5,
                                 float a6, float a7, float a8) {
    M3 r;
    r.m[0][0] = a0; r.m[0][1] = a1; r.m[0][2] = a2;
    r.m[1][0] = a3; r.m[1][1] = a4; r.m[1][2] = a5;
    r.m[2][0] = a6; r.m[2][1] = a7; r.m[2][2] = a8;
    return r;
}

__device__ __forceinline__ M3 mul(const M3 &a, const M3 &b) {
    GSV_NO_CONTRACT
    M3 r;
#pragma unroll
    for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int row = 0; row < 3; ++row)
            r.m[c][row] = a.m[0][row] * b.m[c][0] + a.m[1][row] * b.m[c][1] + a.m[2][row] * b.m[c][2];
    return r;
}

__device__ __forceinline__ M3 transpose(const M3 &a) {
    M3 r;
#pragma unroll
    for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int row = 0; row < 3; ++row) r.m[c][row] = a.m[row][c];
    return r;
}

// Normalised quaternion components (w,x,y,z) from storage [w,x,y,z]; the squared
// norm is summed in the reference's float4 read order (.w,.x,.y,.z).
struct Quat {
    float w, x, y, z;
};
__device__ __forceinline__ Quat unit_quat(float q0, float q1, float q2, float q3) {
    GSV_NO_CONTRACT
    const float n2 = q3 * q3 + q0 * q0 + q1 * q1 + q2 * q2;
    const float s = 1.0f / sqrtf(n2);
    return Quat{q0 * s, q1 * s, q2 * s, q3 * s};
}

// quat_to_rotmat, optim_to_render_helpers.cuh:15-36 (column-major result).
__device__ __forceinline__ M3 rotation(const Quat &q) {
    GSV_NO_CONTRACT
    const float w = q.w, x = q.x, y = q.y, z = q.z;
    return m3(1.f - 2.f * (y * y + z * z), 2.f * (x * y - w * z), 2.f * (x * z + w * y),
              2.f * (x * y + w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z - w * x),
              2.f * (x * z - w * y), 2.f * (y * z + w * x), 1.f - 2.f * (x * x + y * y));
}

struct Geometry {
    M3 R, S, M2, cov;  // cov in voxel units
};

// optim_to_render.cu:85-103 (forward) / 280-300 (backward).  vs = voxel size in
// the kernel's (z, y, x) order, i.e. vs.x belongs to depth.
__device__ __forceinline__ Geometry voxel_geometry(float sx, float sy, float sz, const Quat &q,
                                                   float vsx, float vsy, float vsz) {
    GSV_NO_CONTRACT
    Geometry g;
    g.S = m3(1.f, 0.f, 0.f, 0.f, 1.f, 0.f, 0.f, 0.f, 1.f);
    g.S.m[0][0] = sx;
    g.S.m[1][1] = sy;
    g.S.m[2][2] = sz;
    g.R = rotation(q);
    const M3 M = mul(g.S, g.R);
    M3 cov = mul(transpose(M), M);
    g.M2 = m3(1.f / vsz, 0.0f, 0.0f, 0.0f, 1.f / vsy, 0.0f, 0.0f, 0.0f, 1.f / vsx);
    cov = mul(transpose(g.M2), cov);
    g.cov = mul(cov, g.M2);
    return g;
}

template <int C>
__global__ __launch_bounds__(256) void k_project_fwd(
    int n, const float *__restrict__ pos3d, const float *__restrict__ scale3d,
    const float *__restrict__ quat, const float *__restrict__ intens, int D, int H, int W,
    float wz, float wy, float wx, float cz, float cy, float cx, float4 *__restrict__ pos_radii,
    float *__restrict__ conics, int *__restrict__ tile_min, int *__restrict__ tile_max,
    int *__restrict__ num_tiles_hit) {
    GSV_NO_CONTRACT
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n) return;
    const int Tx = gsv_tiles_along(W), Ty = gsv_tiles_along(H), Tz = gsv_tiles_along(D);
    const float vsx = wz / (float)D, vsy = wy / (float)H, vsz = wx / (float)W;

    const float p0 = pos3d[3 * g + 0], p1 = pos3d[3 * g + 1], p2 = pos3d[3 * g + 2];
    const float s0 = scale3d[3 * g + 0], s1 = scale3d[3 * g + 1], s2 = scale3d[3 * g + 2];
    const float4 q4 = reinterpret_cast<const float4 *>(quat)[g];
    float I[C];
#pragma unroll
    for (int c = 0; c < C; ++c) I[c] = intens[(size_t)g * C + c];

    const float pixx = (p0 - cx + (wx * 0.5f)) / vsz;
    const float pixy = (p1 - cy + (wy * 0.5f)) / vsy;
    const float pixz = (p2 - cz + (wz * 0.5f)) / vsx;

    const Geometry geo = voxel_geometry(s0, s1, s2, unit_quat(q4.x, q4.y, q4.z, q4.w), vsx, vsy, vsz);
    const M3 &cov = geo.cov;
    const float a = cov.m[0][0], b = cov.m[0][1], c = cov.m[0][2];
    const float d = cov.m[1][1], e = cov.m[1][2], f = cov.m[2][2];
    const float det = a * d * f + 2 * b * c * e - a * e * e - f * b * b - d * c * c;

    bool keep = det != 0.0f;
    float ia = 0.f, ib = 0.f, ic = 0.f, id = 0.f, ie = 0.f, iff = 0.f, radius = 0.f;
    int3 tmn = make_int3(0, 0, 0), tmx = make_int3(0, 0, 0);
    int tile_vol = 0;
    if (keep) {
        const float inv_det = 1.0f / det;
        ia = inv_det * (d * f - e * e);
        ib = inv_det * (c * e - b * f);
        ic = inv_det * (b * e - c * d);
        id = inv_det * (a * f - c * c);
        ie = inv_det * (b * c - a * e);
        iff = inv_det * (a * d - b * b);
        radius = ceilf((3.f * fmaxf(s0, fmaxf(s1, s2))) / fminf(vsz, fminf(vsy, vsx)));
        float mean = 0.f;
#pragma unroll
        for (int ch = 0; ch < C; ++ch) mean += I[ch];
        mean /= (float)C;
        const float opt = gsv_logf(mean * GSV_ALPHA_THRESHOLD);
        const float extent = fminf(3.f, sqrtf(2.0f * opt));
        const float r3x = fmaxf(0.0f, (sqrtf(cov.m[0][0]) * extent) - 0.5f);
        const float r3y = fmaxf(0.0f, (sqrtf(cov.m[1][1]) * extent) - 0.5f);
        const float r3z = fmaxf(0.0f, (sqrtf(cov.m[2][2]) * extent) - 0.5f);
        keep = !(radius <= 0.f || pixx + radius < 0.f || pixx - radius > (float)W ||
                 pixy + radius < 0.f || pixy - radius > (float)H || pixz + radius < 0.f ||
                 pixz - radius > (float)D);
        if (keep) {
            const float t = (float)GSV_TILE, t1 = (float)(GSV_TILE - 1);
            tmn.x = gsv_imin(Tx, gsv_imax(0, gsv_f2i_sat((pixx - r3x) / t)));
            tmn.y = gsv_imin(Ty, gsv_imax(0, gsv_f2i_sat((pixy - r3y) / t)));
            tmn.z = gsv_imin(Tz, gsv_imax(0, gsv_f2i_sat((pixz - r3z) / t)));
            tmx.x = gsv_imin(Tx, gsv_imax(0, gsv_f2i_sat((pixx + r3x + t1) / t)));
            tmx.y = gsv_imin(Ty, gsv_imax(0, gsv_f2i_sat((pixy + r3y + t1) / t)));
            tmx.z = gsv_imin(Tz, gsv_imax(0, gsv_f2i_sat((pixz + r3z + t1) / t)));
            tile_vol = (tmx.x - tmn.x) * (tmx.y - tmn.y) * (tmx.z - tmn.z);
            keep = tile_vol > 0;
        }
    }
    if (!keep) {
        ia = ib = ic = id = ie = iff = 0.f;
        tmn = make_int3(0, 0, 0);
        tmx = make_int3(0, 0, 0);
        tile_vol = 0;
    }
    pos_radii[g] = keep ? make_float4(pixx, pixy, pixz, radius) : make_float4(0.f, 0.f, 0.f, 0.f);
    float2 *cn = reinterpret_cast<float2 *>(conics + 6 * (size_t)g);
    cn[0] = make_float2(ia, ib);
    cn[1] = make_float2(ic, id);
    cn[2] = make_float2(ie, iff);
    tile_min[3 * g + 0] = tmn.x; tile_min[3 * g + 1] = tmn.y; tile_min[3 * g + 2] = tmn.z;
    tile_max[3 * g + 0] = tmx.x; tile_max[3 * g + 1] = tmx.y; tile_max[3 * g + 2] = tmx.z;
    num_tiles_hit[g] = tile_vol;
}

// get_cov_grad, optim_to_render.cu:186-239: dL/d(world covariance) from
// dL/d(conic) through the adjugate inverse, with the 1e-7 regulariser.
__device__ __forceinline__ M3 cov_grad(const M3 &cov, const M3 &M2, float gA, float gB, float gC,
                                       float gD, float gE, float gF) {
    GSV_NO_CONTRACT
    const float a = cov.m[0][0], b = cov.m[0][1], c = cov.m[0][2];
    const float d = cov.m[1][1], e = cov.m[1][2], f = cov.m[2][2];
    const float den = a * d * f + 2 * b * c * e - a * e * e - f * b * b - d * c * c;
    const float den2inv = 1.0f / ((den * den) + 0.0000001f);
    M3 out = m3(0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f);
    if (den2inv != 0) {
        const float k_a = d * f - e * e;
        const float k_b = 2 * c * e - 2 * f * b;
        const float k_c = 2 * b * e - 2 * d * c;
        const float k_d = a * f - c * c;
        const float k_e = 2 * b * c - 2 * a * e;
        const float k_f = a * d - b * b;
        const float n_b = c * e - b * f;
        const float n_c = b * e - c * d;
        const float n_e = b * c - a * e;
        const float da = den2inv * (-k_a * k_a * gA - n_b * k_a * gB - n_c * k_a * gC +
                                    (f * den - k_d * k_a) * gD + (-e * den - n_e * k_a) * gE +
                                    (d * den - k_f * k_a) * gF);
        const float db = den2inv * (-k_a * k_b * gA + (-f * den - n_b * k_b) * gB +
                                    (e * den - n_c * k_b) * gC - k_d * k_b * gD +
                                    (c * den - n_e * k_b) * gE + (-2 * b * den - k_f * k_b) * gF);
        const float dc = den2inv * (-k_a * k_c * gA + (e * den - n_b * k_c) * gB +
                                    (-d * den - n_c * k_c) * gC + (-2 * c * den - k_d * k_c) * gD +
                                    (b * den - n_e * k_c) * gE - k_f * k_c * gF);
        const float dd = den2inv * ((f * den - k_a * k_d) * gA - n_b * k_d * gB +
                                    (-c * den - n_c * k_d) * gC - k_d * k_d * gD - n_e * k_d * gE +
                                    (a * den - k_f * k_d) * gF);
        const float de = den2inv * ((-2 * e * den - k_a * k_e) * gA + (c * den - n_b * k_e) * gB +
                                    (b * den - n_c * k_e) * gC - k_d * k_e * gD +
                                    (-a * den - n_e * k_e) * gE + -k_f * k_e * gF);
        const float df = den2inv * ((d * den - k_a * k_f) * gA + (-b * den - n_b * k_f) * gB -
                                    n_c * k_f * gC + (a * den - k_d * k_f) * gD - n_e * k_f * gE -
                                    k_f * k_f * gF);
        const M3 dhat = m3(da, db, dc, db, dd, de, dc, de, df);
        const M3 t = mul(mul(M2, dhat), transpose(M2));
#pragma unroll
        for (int col = 0; col < 3; ++col)
#pragma unroll
            for (int row = 0; row < 3; ++row) out.m[col][row] = 0.5f * (t.m[col][row] + t.m[row][col]);
    }
    return out;
}

__global__ __launch_bounds__(256) void k_project_bwd(
    int n, const float *__restrict__ scale3d, const float *__restrict__ quat, int D, int H, int W,
    float wz, float wy, float wx, const float4 *__restrict__ dpos_radii,
    const float *__restrict__ dconics, const float4 *__restrict__ pos_radii,
    float *__restrict__ dpos, float *__restrict__ dscale, float *__restrict__ dquat) {
    GSV_NO_CONTRACT
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n) return;
    float out_p[3] = {0.f, 0.f, 0.f}, out_s[3] = {0.f, 0.f, 0.f}, out_q[4] = {0.f, 0.f, 0.f, 0.f};
    if (!(pos_radii[g].w <= 0)) {
        const float vsx = wz / (float)D, vsy = wy / (float)H, vsz = wx / (float)W;
        const float s0 = scale3d[3 * g + 0], s1 = scale3d[3 * g + 1], s2 = scale3d[3 * g + 2];
        const float4 q4 = reinterpret_cast<const float4 *>(quat)[g];
        const Quat q = unit_quat(q4.x, q4.y, q4.z, q4.w);
        const Geometry geo = voxel_geometry(s0, s1, s2, q, vsx, vsy, vsz);
        const float *gc = dconics + 6 * (size_t)g;
        const M3 cg = cov_grad(geo.cov, geo.M2, gc[0], gc[1], gc[2], gc[3], gc[4], gc[5]);
        const M3 dsig = m3(cg.m[0][0], 0.5f * cg.m[0][1], 0.5f * cg.m[0][2], 0.5f * cg.m[1][0],
                           cg.m[1][1], 0.5f * cg.m[1][2], 0.5f * cg.m[2][0], 0.5f * cg.m[2][1],
                           cg.m[2][2]);
        M3 S2;
#pragma unroll
        for (int col = 0; col < 3; ++col)
#pragma unroll
            for (int row = 0; row < 3; ++row) S2.m[col][row] = 2.0f * geo.S.m[col][row];
        const M3 Rg = mul(mul(S2, geo.R), dsig);
        M3 Rgt = transpose(Rg);
        const M3 Rt = transpose(geo.R);
#pragma unroll
        for (int i = 0; i < 3; ++i)
            out_s[i] = Rt.m[i][0] * Rgt.m[i][0] + Rt.m[i][1] * Rgt.m[i][1] + Rt.m[i][2] * Rgt.m[i][2];
        const float sc[3] = {s0, s1, s2};
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int row = 0; row < 3; ++row) Rgt.m[i][row] *= sc[i];
        const float4 dp = dpos_radii[g];
        out_p[0] = dp.x * vsz;
        out_p[1] = dp.y * vsy;
        out_p[2] = dp.z * vsx;
        // rotmat_grad_to_quat_grad, optim_to_render_helpers.cuh:51-75
        const float w = q.w, x = q.x, y = q.y, z = q.z;
        const float(*v)[3] = Rgt.m;
        out_q[0] = 2 * z * (v[0][1] - v[1][0]) + 2 * y * (v[2][0] - v[0][2]) + 2 * x * (v[1][2] - v[2][1]);
        out_q[1] = 2 * y * (v[1][0] + v[0][1]) + 2 * z * (v[2][0] + v[0][2]) +
                   2 * w * (v[1][2] - v[2][1]) - 4 * x * (v[2][2] + v[1][1]);
        out_q[2] = 2 * x * (v[1][0] + v[0][1]) + 2 * w * (v[2][0] - v[0][2]) +
                   2 * z * (v[1][2] + v[2][1]) - 4 * y * (v[2][2] + v[0][0]);
        out_q[3] = 2 * w * (v[0][1] - v[1][0]) + 2 * x * (v[2][0] + v[0][2]) +
                   2 * y * (v[1][2] + v[2][1]) - 4 * z * (v[1][1] + v[0][0]);
    }
    dpos[3 * g + 0] = out_p[0]; dpos[3 * g + 1] = out_p[1]; dpos[3 * g + 2] = out_p[2];
    dscale[3 * g + 0] = out_s[0]; dscale[3 * g + 1] = out_s[1]; dscale[3 * g + 2] = out_s[2];
    reinterpret_cast<float4 *>(dquat)[g] = make_float4(out_q[0], out_q[1], out_q[2], out_q[3]);
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace gsv

using namespace gsv;

extern "C" int gsv_project_fwd(int32_t n, int32_t channels, const float *pos3d,
                               const float *scale3d, const float *quat, const float *intensities,
                               int32_t D, int32_t H, int32_t W, float world_z, float world_y,
                               float world_x, float center_z, float center_y, float center_x,
                               float *pos3d_radii, float *conics, int32_t *tile_min,
                               int32_t *tile_max, int32_t *num_tiles_hit, void *stream) {
    if (channels < 1 || channels > GSV_MAX_CHANNELS) return GSV_ERR_UNSUPPORTED_CHANNELS;
    if (n < 0 || D <= 0 || H <= 0 || W <= 0) return GSV_ERR_INVALID_ARGUMENT;
    if (n == 0) return GSV_OK;
    if (!pos3d || !scale3d || !quat || !intensities || !pos3d_radii || !conics || !tile_min ||
        !tile_max || !num_tiles_hit)
        return GSV_ERR_INVALID_ARGUMENT;
    if (!aligned(quat, 16) || !aligned(pos3d_radii, 16) || !aligned(conics, 8))
        return GSV_ERR_INVALID_ARGUMENT;
    const dim3 grid((n + 255) / 256), block(256);
    hipStream_t s = as_stream(stream);
#define GSV_PF(CH)                                                                               \
    hipLaunchKernelGGL(k_project_fwd<CH>, grid, block, 0, s, n, pos3d, scale3d, quat,            \
                       intensities, D, H, W, world_z, world_y, world_x, center_z, center_y,      \
                       center_x, reinterpret_cast<float4 *>(pos3d_radii), conics, tile_min,      \
                       tile_max, num_tiles_hit)
    switch (channels) {
        case 1: GSV_PF(1); break;
        case 2: GSV_PF(2); break;
        case 3: GSV_PF(3); break;
        default: GSV_PF(4); break;
    }
#undef GSV_PF
    return check_launch();
}

extern "C" int gsv_project_bwd(int32_t n, const float *pos3d, const float *scale3d,
                               const float *quat, int32_t D, int32_t H, int32_t W, float world_z,
                               float world_y, float world_x, float center_z, float center_y,
                               float center_x, const float *dpos3d_radii, const float *dconics,
                               const float *pos3d_radii, float *dpos3d, float *dscale3d,
                               float *dquat, void *stream) {
    (void)pos3d; (void)center_z; (void)center_y; (void)center_x;
    if (n < 0 || D <= 0 || H <= 0 || W <= 0) return GSV_ERR_INVALID_ARGUMENT;
    if (n == 0) return GSV_OK;
    if (!scale3d || !quat || !dpos3d_radii || !dconics || !pos3d_radii || !dpos3d || !dscale3d ||
        !dquat)
        return GSV_ERR_INVALID_ARGUMENT;
    if (!aligned(quat, 16) || !aligned(dpos3d_radii, 16) || !aligned(pos3d_radii, 16) ||
        !aligned(dquat, 16))
        return GSV_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_project_bwd, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), n,
                       scale3d, quat, D, H, W, world_z, world_y, world_x,
                       reinterpret_cast<const float4 *>(dpos3d_radii), dconics,
                       reinterpret_cast<const float4 *>(pos3d_radii), dpos3d, dscale3d, dquat);
    return check_launch();
}
