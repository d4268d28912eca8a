/*
 * gsvox.h — C ABI of libgsvox.so, the gfx950 Gaussian voxelizer.
 *
 * Drop-in boundary for the reference's native module `gs_voxelizer.cuda`
 * (PaPieta/gs-voxelizer v0.1.0, gs_voxelizer/cuda/ext.cpp:4-11, signatures in
 * gs_voxelizer/cuda/bindings.h:40-194).  The reference binds torch tensors with
 * pybind11 and allocates its outputs; this ABI takes plain device pointers and
 * sizes instead, the caller allocates every output and workspace, and each call
 * only enqueues work on `stream` (a hipStream_t; NULL = the default stream).
 *
 * Conventions shared by every entry point
 *   - Volume tuples are (z, y, x) = (D, H, W); pos3d / scale3d / tile indices
 *     are (x, y, z); quat is [w, x, y, z]; the volume is (D, H, W, C) row-major.
 *   - All arrays are contiguous, device-resident, 4-byte aligned; pos3d_radii
 *     rows are float4 (16-byte aligned); conics rows are 6 floats (8-byte aligned).
 *   - Return value: GSV_OK (0) or a gsv_status code; nothing is ever printed and
 *     the process is never terminated.  A HIP launch error is reported as
 *     GSV_ERR_HIP; gsv_last_hip_error() returns the underlying hipError_t.
 *   - Outputs are fully written (zero where the reference zero-fills) with
 *     kernels, never hipMemset, so a caller may capture the calls in a graph.
 *   - Calls are stateless and may be issued from any host thread; calls on one
 *     stream execute in order.
 */
#ifndef GSVOX_H
#define GSVOX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum gsv_status {
    GSV_OK = 0,
    GSV_ERR_INVALID_ARGUMENT = 1,   /* negative size, NULL pointer, bad variant */
    GSV_ERR_UNSUPPORTED_CHANNELS = 2, /* channels outside [1, 4] (bindings.cu:61-63) */
    GSV_ERR_WORKSPACE_TOO_SMALL = 3,
    GSV_ERR_SIZE_OVERFLOW = 4,      /* an index would not fit the int32 layout */
    GSV_ERR_HIP = 5,                /* a HIP runtime call or launch failed */
    GSV_ERR_SCRATCH_TOO_SMALL = 6   /* beyond the fixed scratch of gsv_bin_and_sort_noalloc */
} gsv_status;

/* Library version, MAJOR*10000 + MINOR*100 + PATCH. */
int gsv_version(void);

/* Human-readable text for a gsv_status value (static storage). */
const char *gsv_status_string(int status);

/* hipError_t of the most recent failing HIP call made by this thread. */
int gsv_last_hip_error(void);

/*
 * Projection forward: optimisation parameters -> rendering parameters.
 * Replaces optim_to_render_forward_torch (bindings.cu:38-189; kernel
 * optim_to_render.cu:48-172).  Outputs per Gaussian: pos3d_radii (n,4) = voxel
 * position xyz + integer-valued radius, conics (n,6) = inverse covariance
 * (00,01,02,11,12,22) in voxel units, tile_min / tile_max (n,3) int32 [min, max)
 * tile box, num_tiles_hit (n,) int32.  Culled Gaussians get all-zero rows.
 * intensities is (n, channels); channels in [1, 4].
 */
int gsv_project_fwd(int32_t n, int32_t channels, const float *pos3d, const float *scale3d,
                    const float *quat, const float *intensities, int32_t D, int32_t H, int32_t W,
                    float world_z, float world_y, float world_x, float center_z, float center_y,
                    float center_x, float *pos3d_radii, float *conics, int32_t *tile_min,
                    int32_t *tile_max, int32_t *num_tiles_hit, void *stream);

/*
 * Projection backward.  Replaces optim_to_render_backward_torch
 * (bindings.cu:197-251; kernel optim_to_render.cu:246-336).  Gradients w.r.t.
 * pos3d (n,3), scale3d (n,3), quat (n,4) from the gradients of pos3d_radii (n,4)
 * and conics (n,6); rows whose pos3d_radii[:,3] <= 0 get zeros.  Same formulas
 * as the reference: dpos = dpix * voxel_size, dquat without the normalisation
 * Jacobian, 1e-7 regulariser on det^2.
 */
int gsv_project_bwd(int32_t n, const float *pos3d, const float *scale3d, const float *quat,
                    int32_t D, int32_t H, int32_t W, float world_z, float world_y, float world_x,
                    float center_z, float center_y, float center_x, const float *dpos3d_radii,
                    const float *dconics, const float *pos3d_radii, float *dpos3d,
                    float *dscale3d, float *dquat, void *stream);

/*
 * Inclusive int32 prefix sum of num_tiles_hit.  Replaces the
 * `torch.cumsum(num_tiles_hit, dim=0, dtype=torch.int32)` of voxelize.py:87.
 * If total_out is non-NULL the last element (the intersection count) is also
 * written to that device int64, so a caller can read one scalar.  If
 * total_host is non-NULL it must be pinned host memory (hipHostMalloc, or a
 * torch tensor made with pin_memory=True): the kernel writes the count there
 * too, visible to the host once the scan has completed (e.g. after an event
 * recorded behind this call), so no device-to-host copy is enqueued.  A
 * total_host that is not device-visible pinned memory returns
 * GSV_ERR_INVALID_ARGUMENT.  Workspace size from gsv_scan_workspace_bytes.
 */
int gsv_scan_workspace_bytes(int64_t n, size_t *bytes);
int gsv_cumsum_tiles_hit(int32_t n, const int32_t *num_tiles_hit, int32_t *cum_tiles_hit,
                         int64_t *total_out, int64_t *total_host, void *workspace,
                         size_t workspace_bytes, void *stream);

/*
 * Binning.  Replaces bin_and_sort_gaussians_torch (bindings.cu:259-360):
 * map_gaussian_to_intersects (bin_and_sort_gaussians.cu:11-35), the stable
 * 32-bit CUB radix sort (bindings.cu:313-345) and get_tile_bin_edges
 * (bin_and_sort_gaussians.cu:40-62).  Outputs gaussian_ids_sorted (I,) int32,
 * ordered by (tile id, gaussian id), and tile_bins (T,2) int32 [start, end)
 * with (0,0) for empty tiles, T = ceil(W/8)*ceil(H/8)*ceil(D/8).
 * cum_tiles_hit is the inclusive scan of the per-Gaussian tile counts and must
 * end at num_intersects.  num_intersects <= 0 only zero-fills tile_bins.
 * tiles_sorted (optional, NULL to skip; num_intersects entries, 16-byte
 * aligned) receives the sorted keys: the tile id of each sorted pair, which
 * gsv_voxelize_bwd can take instead of rebuilding it from tile_bins.  The
 * reference keeps these keys in a scratch tensor (bindings.cu:295-345).
 * The library sorts with one of two methods of equal result (a top-digit
 * split into per-bucket sorts, or LSD radix passes), chosen by the key width,
 * the pair count and the Gaussian count; the environment variable
 * GSV_BINNING=lsd or =bucket overrides the choice (for tests).  The workspace
 * size does not depend on it.
 */
int gsv_bin_workspace_bytes(int32_t n, int64_t num_intersects, int32_t D, int32_t H, int32_t W,
                            size_t *bytes);
int gsv_bin_and_sort(int32_t n, int64_t num_intersects, const int32_t *tile_min,
                     const int32_t *tile_max, const int32_t *cum_tiles_hit, int32_t D, int32_t H,
                     int32_t W, void *workspace, size_t workspace_bytes,
                     int32_t *gaussian_ids_sorted, int32_t *tile_bins, int32_t *tiles_sorted,
                     void *stream);

/*
 * Binning with the pair count left on the device.  Replaces the same reference
 * path as gsv_bin_and_sort, minus the host read of the count
 * (voxelize.py:87-88, `cum_tiles_hit[-1].item()`).  The kernels read the live
 * count I = *num_intersects_dev (an int64, e.g. the total written by
 * gsv_cumsum_tiles_hit) and sort min(I, capacity) pairs.  Grids, the workspace
 * (gsv_bin_workspace_bytes with num_intersects = capacity) and
 * gaussian_ids_sorted and tiles_sorted (capacity entries each, 16-byte
 * aligned; tiles_sorted optional) are sized by capacity.  When I > capacity
 * the output is incomplete: the caller compares I with capacity once the count
 * reaches the host, and runs again with a larger capacity.
 */
int gsv_bin_and_sort_device_count(int32_t n, int64_t capacity, const int64_t *num_intersects_dev,
                                  const int32_t *tile_min, const int32_t *tile_max,
                                  const int32_t *cum_tiles_hit, int32_t D, int32_t H, int32_t W,
                                  void *workspace, size_t workspace_bytes,
                                  int32_t *gaussian_ids_sorted, int32_t *tile_bins,
                                  int32_t *tiles_sorted, void *stream);

/*
 * Prefix sum and binning in one call, with the pair count left on the device.
 * Replaces voxelize.py:87-88 and bin_and_sort_gaussians_torch
 * (bindings.cu:259-360): the same work and outputs as gsv_cumsum_tiles_hit
 * (cum_tiles_hit, *total_out, *total_host as described there) followed by
 * gsv_bin_and_sort_device_count with num_intersects_dev = total_out.
 * total_out is required.  Workspace size from gsv_cumsum_bin_workspace_bytes
 * (n, capacity, D, H, W).  Where the binning takes the bucket method with a
 * single-pass scan of its block sums (n up to 4,194,304), the bucket counts
 * are formed beside the scan's block sums and their prefix beside the scan's
 * apply pass: four kernel launches instead of six, the same results.  When
 * *total_out > capacity, only *total_out (and *total_host, cum_tiles_hit) is
 * valid: gaussian_ids_sorted, tile_bins and tiles_sorted may hold any values
 * (on the bucket method they are not a sorted prefix, unlike
 * gsv_bin_and_sort_device_count's); the caller bins again with a capacity of
 * at least the count.  Every access stays inside the arrays, also when the
 * count passes 2^31.
 */
int gsv_cumsum_bin_workspace_bytes(int32_t n, int64_t capacity, int32_t D, int32_t H, int32_t W,
                                   size_t *bytes);
int gsv_cumsum_bin_and_sort_device_count(int32_t n, int64_t capacity,
                                         const int32_t *num_tiles_hit, const int32_t *tile_min,
                                         const int32_t *tile_max, int32_t D, int32_t H, int32_t W,
                                         int32_t *cum_tiles_hit, int64_t *total_out,
                                         int64_t *total_host, void *workspace,
                                         size_t workspace_bytes, int32_t *gaussian_ids_sorted,
                                         int32_t *tile_bins, int32_t *tiles_sorted, void *stream);

/*
 * Binning that allocates nothing.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory when they bin (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, outputs and results as gsv_bin_and_sort without the workspace:
 * the kernels use a fixed array in device memory that the library owns, one per
 * GPU, 52,431,104 bytes (50 MiB), held until the process ends.
 * It holds problems of up to GSV_NOALLOC_MAX_INTERSECTIONS (tile, Gaussian)
 * pairs (the 256^3 / 200,000-Gaussian scene has 3.54 M); a larger
 * num_intersects returns GSV_ERR_SCRATCH_TOO_SMALL before anything is enqueued.
 * The stream must belong to the current device.  No part of the array needs
 * to start at zero: each call writes what it reads.  Every call on one GPU
 * uses that GPU's single array, so calls that overlap in time on one GPU
 * (other streams, other host threads) race; the caller serialises them.
 */
#define GSV_NOALLOC_MAX_INTERSECTIONS 4194304
int gsv_bin_and_sort_noalloc(int32_t n, int64_t num_intersects, const int32_t *tile_min,
                             const int32_t *tile_max, const int32_t *cum_tiles_hit, int32_t D,
                             int32_t H, int32_t W, int32_t *gaussian_ids_sorted,
                             int32_t *tile_bins, int32_t *tiles_sorted, void *stream);

/*
 * Forward voxelization.  Replaces voxelize_forward_torch (bindings.cu:362-457;
 * kernel voxelize.cu:39-164).  volume (D,H,W,channels) float32 is fully written.
 * n = number of Gaussians (rows of pos3d_radii / conics / intensities).
 * pair_live (optional, num_intersects bytes, one per sorted pair): receives 1
 * for every pair the kernel evaluated and 0 for each it culled, i.e. whose
 * tile holds no voxel centre inside the Gaussian's gate ellipsoid (such a pair
 * adds nothing to the volume).  Handing it to the backward lets that skip the
 * culled pairs too.
 */
int gsv_voxelize_fwd(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                     int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                     const int32_t *tile_bins, const float *pos3d_radii, const float *conics,
                     const float *intensities, float *volume, uint8_t *pair_live,
                     void *stream);

/*
 * Backward voxelization.  Replaces voxelize_backward_per_gaussian_torch
 * (bindings.cu:586-781; kernel voxelize.cu:368-574) when variant = 1 and
 * voxelize_backward_torch (bindings.cu:459-584; kernel voxelize.cu:170-366)
 * when variant = 0.  Both variants compute the same gradients (up to float
 * summation order); this library serves both with one kernel.  Outputs
 * dpos3d_radii (n,4) (column 3 stays 0), dconics (n,6), dintensities
 * (n,channels), all fully written.  No host synchronisation happens inside.
 *
 * Reduction across tiles:
 *   - tile_min, tile_max, cum_tiles_hit all NULL: float atomics (the
 *     reference's scheme; summation order, hence the last bits, vary run to run);
 *   - all three given (the projection's tile boxes and the prefix sum the
 *     binning used): each (tile, Gaussian) pair writes its partial gradient to
 *     its duplication slot and one pass sums each Gaussian's slots in order.
 *     No atomics, and the same bits from run to run on the same inputs; the
 *     workspace grows by num_intersects * (9 + channels) * 4 bytes.
 * tiles_sorted (optional) is the binning's sorted keys (gsv_bin_and_sort's
 * tiles_sorted, at least num_intersects entries); without it the tile of each
 * pair is rebuilt from tile_bins by one more kernel.
 * num_intersects_dev (optional, device int64): the live pair count, as left by
 * gsv_cumsum_tiles_hit; num_intersects is then the capacity that the id, tile
 * and workspace arrays and the grids are sized for (gsv_bin_and_sort_device_count
 * outputs), and the kernels process min(count, capacity) pairs.  With it the
 * backward needs no host-side count, so a caller can capture it in a graph.
 * pair_live (optional): the flags the forward wrote (gsv_voxelize_fwd's
 * pair_live, same pairs); the backward then evaluates only the pairs the
 * forward kept and gives the culled ones a zero partial.  With chained rows
 * off (gsv_set_backward_chains(0) or GSV_BWD_CHAIN=0) the gradients are the
 * same bits as without it.  With them on (the default) a group of 64 pairs
 * takes the chained rows only when all of its pairs qualify, so a pair's
 * rounding depends on the pairs that share its wave, and the flags, the
 * capacity mode and the tile map change that grouping: the results then agree
 * to rounding (rel 1e-4 / abs 1e-6), not bit for bit.
 * Workspace size from gsv_voxelize_bwd_workspace_bytes (n = the Gaussian
 * count, deterministic = 1 for the second mode): besides the per-pair arrays
 * it holds one 128-byte record per Gaussian, which a first kernel fills with
 * what the pairs read of their Gaussian and the parts of their set-up that do
 * not depend on the tile (the gate, the binary64 factor of the conic, the
 * chain bounds' Gaussian terms, the column factors, the emission box).
 */
int gsv_voxelize_bwd_workspace_bytes(int32_t D, int32_t H, int32_t W, int32_t channels,
                                     int32_t n, int64_t num_intersects, int32_t deterministic,
                                     size_t *bytes);
int gsv_voxelize_bwd(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                     int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                     const int32_t *tile_bins, const float *pos3d_radii, const float *conics,
                     const float *intensities, const float *vol_grad, const int32_t *tile_min,
                     const int32_t *tile_max, const int32_t *cum_tiles_hit,
                     const int32_t *tiles_sorted, const int64_t *num_intersects_dev,
                     const uint8_t *pair_live, float *dpos3d_radii, float *dconics,
                     float *dintensities, int32_t variant, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * Chained rows of the backward (no counterpart in the reference).  The
 * backward forms most exp2 values of a tile row as products of two or three
 * v_exp_f32 results when every pair of a 64-pair group allows it; that is
 * faster and equal to the per-voxel evaluation to rounding, but makes a pair's
 * last bits depend on its group (see pair_live above).  enabled = 0 turns the
 * chains off for every later backward of the process (bitwise reproducible
 * across culling and capacity modes), 1 turns them on; *previous (optional)
 * receives the setting before the call.  The first backward of a process
 * takes the setting from GSV_BWD_CHAIN (off when "0") unless this was called
 * before; the variable is read only then.
 */
int gsv_set_backward_chains(int32_t enabled, int32_t *previous);

/*
 * Voxelization fused with an L1 loss.  These have no reference binding.  They
 * fuse the voxelizer with the loss of the reference's training loop (README.md:77-82,
 * torch.nn.functional.l1_loss with reduction "mean") so that dL/dvolume is
 * never materialised.
 *
 * gsv_voxelize_fwd_l1: gsv_voxelize_fwd plus *loss (one float on the device)
 * = mean over all D*H*W*channels elements of |volume - target|, target laid
 * out like volume.  The loss is summed per tile in binary32 and over tiles in
 * binary64 in a fixed order.  `sign` (int8, laid out like volume) receives
 * sgn(volume - target): -1, 0 or 1, and 0 where the difference is NaN (torch's
 * sign of NaN, so the backward matches l1_loss's there too; the loss is NaN).
 * pair_live as for gsv_voxelize_fwd.
 * Workspace: gsv_voxelize_fwd_l1_workspace_bytes.
 *
 * gsv_voxelize_bwd_l1: gsv_voxelize_bwd with vol_grad replaced by
 * sign * (*grad_loss * (1 / numel)), exactly what torch's l1_loss backward
 * produces, plus vol_grad when it is not NULL (the volume's gradient from
 * other uses).  grad_loss is one float on the device.  Same workspace and
 * reduction modes as gsv_voxelize_bwd.
 */
int gsv_voxelize_fwd_l1_workspace_bytes(int32_t D, int32_t H, int32_t W, size_t *bytes);
int gsv_voxelize_fwd_l1(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                        int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                        const int32_t *tile_bins, const float *pos3d_radii, const float *conics,
                        const float *intensities, const float *target, float *volume,
                        int8_t *sign, float *loss, uint8_t *pair_live, void *workspace,
                        size_t workspace_bytes, void *stream);
int gsv_voxelize_bwd_l1(int32_t D, int32_t H, int32_t W, int32_t channels, int32_t n,
                        int64_t num_intersects, const int32_t *gaussian_ids_sorted,
                        const int32_t *tile_bins, const float *pos3d_radii, const float *conics,
                        const float *intensities, const int8_t *sign, const float *grad_loss,
                        const float *vol_grad, const int32_t *tile_min, const int32_t *tile_max,
                        const int32_t *cum_tiles_hit, const int32_t *tiles_sorted,
                        const int64_t *num_intersects_dev, const uint8_t *pair_live,
                        float *dpos3d_radii, float *dconics, float *dintensities,
                        int32_t variant, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Kernel timing (no counterpart in the reference; for benchmarks and
 * profiling).  While enabled, each launch of the hot kernels is bracketed by
 * two HIP events recorded on its launch stream.  collect() waits for the
 * recorded events and returns the summed duration and launch count of one
 * kernel since the previous collect: 0 = forward voxelize kernel, 1 = backward
 * voxelize kernel, 2 = backward per-Gaussian reduction.  Off by default; costs
 * nothing when off.
 */
int gsv_kernel_timing_enable(int32_t enable);
int gsv_kernel_timing_collect(int32_t kernel, double *total_ms, int32_t *count);

/*
 * Per-workgroup timeline (no counterpart in the reference; for profiling load
 * balance).  While a buffer is registered, every launch of the forward
 * voxelize kernel (kernel = 0; the only one supported) writes, for each
 * workgroup b < capacity that has a tile, records[3b] = its start and
 * records[3b+1] = its end on the GPU's constant 100 MHz wall clock and
 * records[3b+2] = its tile index.  `records` is the caller's device buffer of
 * 3 * capacity uint64 on the device current at registration, and only launches
 * on that device record; NULL unregisters.  Later launches overwrite earlier
 * ones; the forward launches one workgroup per tile (rounded up to a multiple
 * of 64).  Costs one uniform branch per workgroup when unregistered.
 */
int gsv_wave_timeline(int32_t kernel, uint64_t *records, int32_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* GSVOX_H */
