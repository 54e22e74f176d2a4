/*
 * gsplat_hip.h -- C ABI of the MI355X (gfx950) splatting operator chain.
 *
 * Plain pointers, sizes and a HIP stream (passed as void*); no torch or MLX
 * types. Every pointer is device memory; inputs are read-only and C-contiguous
 * in the reference layouts (AoS float32, int32 radii/offsets/ids, int64 keys).
 * Outputs are caller-allocated; each entry point writes every element of its
 * outputs (including zeros for culled / masked entries), so callers need not
 * clear them. Work is enqueued on `stream` and returns without synchronizing,
 * except where a function says otherwise.
 *
 * Return value: GSPLAT_OK (0) or a GSPLAT_ERR_* code; gsplat_hip_last_error()
 * then returns a message for the calling thread.
 *
 * Each entry point replaces the device half (`eval_gpu`) of one reference MLX
 * primitive, or an MLX library op on the path; the reference file:line of
 * the interface it replaces is given beside it.
 */
#ifndef GSPLAT_HIP_H_
#define GSPLAT_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GSPLAT_OK = 0,
  GSPLAT_ERR_INVALID_ARGUMENT = 1,
  GSPLAT_ERR_HIP = 2,
  GSPLAT_ERR_WORKSPACE_TOO_SMALL = 3,
};

/* Message for the last failing call on this thread ("" if none). */
const char* gsplat_hip_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int gsplat_hip_abi_version(void);

/* Opt-in kernel timing (no counterpart in the reference; used by the
 * benchmark). While enabled, every entry point brackets each kernel it
 * launches with a pair of HIP events recorded on the launch stream.
 * gsplat_hip_profile_report() waits for the recorded events, writes one line
 * "name<TAB>launches<TAB>total_ms" per kernel into buf (NUL-terminated,
 * truncated to buf_len) and returns the length of the full report; it keeps
 * the totals until gsplat_hip_profile_reset(). Not for concurrent use from
 * several host threads. */
void gsplat_hip_profile_enable(int32_t enable);
void gsplat_hip_profile_reset(void);
size_t gsplat_hip_profile_report(char* buf, size_t buf_len);

/* Measurement probe (no counterpart in the reference; used by the
 * benchmark): `blocks` workgroups of 256 lanes each run 8 independent FP32
 * FMA chains of `iters` steps and write one float per lane to out
 * [blocks * 256]. Timed by the caller, it gives the attainable FP32 rate of
 * single (not packed) VALU instructions: blocks * 256 * 8 * 2 * iters flops. */
int gsplat_hip_valu_probe(float* out, int64_t blocks, int32_t iters, void* stream);

/* Measurement probe (no counterpart in the reference; used by the
 * benchmark): the attainable rate of LDS broadcast reads, the rasterizers'
 * record access. `blocks` workgroups of 256 lanes each make `iters` (a
 * multiple of 256) steps of four ds_read_b128 per wave at wave-uniform
 * addresses and write one word per lane to out [blocks * 256]. Timed by the
 * caller: blocks * 4 * iters * 4 wave-level 16-byte broadcast reads. */
int gsplat_hip_lds_probe(uint32_t* out, int64_t blocks, int32_t iters, void* stream);

/* Unit-test probe (no counterpart in the reference): out[i] = the
 * rasterizer's exp(y[i]) for n floats (the exponential behind every alpha of
 * rasterize_fwd / rasterize_bwd / rasterize_to_indices). Equal to expf for
 * y > -103; at most 2^-149 for y <= -104 (including -inf); NaN for NaN. */
int gsplat_hip_exp_alpha_eval(const float* y, int64_t n, float* out, void* stream);

/* ---------------------------------------------------------------------------
 * quat_scale_to_covar_preci
 * Replaces GSPlatQuatScaleToCovarPreci(/Backward)::eval_gpu
 * (gsplat_core/gsplat_quat_scale_to_covar.cpp:470-552,
 *  gsplat_core/include/gsplat_quat_scale_to_covar.h:42-46).
 * quats [n,4] (w,x,y,z), scales [n,3]; covars/precis [n,6] (triu) or [n,3,3];
 * a disabled output may be NULL. Backward: v_covars / v_precis may be NULL
 * (not requested); v_quats [n,4], v_scales [n,3].
 * ------------------------------------------------------------------------- */
int gsplat_hip_quat_scale_to_covar_preci_fwd(const float* quats, const float* scales, int64_t n,
                                             int32_t compute_covar, int32_t compute_preci,
                                             int32_t triu, float* covars, float* precis,
                                             void* stream);
int gsplat_hip_quat_scale_to_covar_preci_bwd(const float* quats, const float* scales,
                                             const float* v_covars, const float* v_precis,
                                             int64_t n, int32_t triu, float* v_quats,
                                             float* v_scales, void* stream);

/* ---------------------------------------------------------------------------
 * Fused EWA projection.
 * Replaces GSPlatProjectionEWA3DGSFused(/Backward)::eval_gpu
 * (gsplat_core/gsplat_projection.cpp:654-855,
 *  gsplat_core/include/gsplat_projection.h:12-77). Field meanings follow
 * ProjectionEWA3DGSFusedParams (gsplat_projection.h:12-23).
 * ------------------------------------------------------------------------- */
typedef struct gsplat_projection_params {
  int32_t image_width;
  int32_t image_height;
  float eps2d;
  float near_plane;
  float far_plane;
  float radius_clip;
  int32_t calc_compensations;
  int32_t camera_model; /* 0 pinhole, 1 orthographic, 2 fisheye (forward and backward) */
  int32_t use_covars;
  int32_t use_opacities;
} gsplat_projection_params;

/* means [B,N,3]; covars [B,N,6] (use_covars) or quats [B,N,4] + scales
 * [B,N,3]; opacities [B,N] (use_opacities, else NULL); viewmats [B,C,4,4]
 * row-major world-to-camera; Ks [B,C,3,3]. Outputs over [B,C,N]: radii
 * (int32, x2), means2d (x2), depths, conics (x3), compensations
 * (calc_compensations, else NULL). */
int gsplat_hip_projection_fwd(const float* means, const float* covars, const float* quats,
                              const float* scales, const float* opacities,
                              const float* viewmats, const float* Ks, int64_t B, int64_t C,
                              int64_t N, const gsplat_projection_params* params,
                              int32_t* radii, float* means2d, float* depths, float* conics,
                              float* compensations, void* stream);

/* Pinhole, orthographic and fisheye (the reference's backward is pinhole
 * only, gsplat_projection.cpp:157-160). Gradients w.r.t. means [B,N,3] and either
 * covars [B,N,6] or quats [B,N,4] + scales [B,N,3] (the other pair NULL);
 * v_viewmats [B,C,4,4] when non-NULL (needs a workspace of
 * gsplat_hip_projection_bwd_workspace_size bytes, else workspace may be NULL).
 * compensations / v_compensations are NULL unless calc_compensations.
 * v_depths may be NULL, meaning zeros (the reference always passes an
 * array; NULL saves the caller a zero fill when its loss ignores depth). */
size_t gsplat_hip_projection_bwd_workspace_size(int64_t B, int64_t C, int64_t N,
                                                int32_t viewmats_grad);
int gsplat_hip_projection_bwd(const float* means, const float* covars, const float* quats,
                              const float* scales, const float* viewmats, const float* Ks,
                              int64_t B, int64_t C, int64_t N,
                              const gsplat_projection_params* params, const int32_t* radii,
                              const float* conics, const float* compensations,
                              const float* v_means2d, const float* v_depths,
                              const float* v_conics, const float* v_compensations,
                              float* v_means, float* v_covars, float* v_quats, float* v_scales,
                              float* v_viewmats, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Packed layout: upstream gsplat's fully_fused_projection(packed=True)
 * (projection_ewa_3dgs_packed_fwd/bwd, note/gsplat_cuda_source_map.md:273-315;
 * the reference's intended projection_ewa_3dgs_packed_forward). Only the
 * visible (camera, Gaussian) pairs are written, nnz of them, in the order of
 * idx = (b * C + c) * N + n; each packed row equals the dense output at idx
 * bit for bit.
 *  count: computes every pair's visibility into the workspace and the count
 *    nnz at *nnz_dev (device int64; the caller reads it to size the outputs).
 *  fwd: with the same workspace, writes batch_ids, camera_ids, gaussian_ids
 *    (int32 [nnz]), indptr [B*C + 1] (first packed row of each camera; the
 *    last is nnz), radii [nnz,2], means2d [nnz,2], depths [nnz], conics
 *    [nnz,3] and compensations [nnz] (calc_compensations, else NULL).
 *  bwd: gradients from the packed cotangents (v_* [nnz, ...]); the packed ids
 *    must be those of the forward (ascending idx, no repeats); batch_ids may
 *    be NULL when B == 1. Outputs as gsplat_hip_projection_bwd, bit for bit
 *    the dense backward with the cotangents scattered to their pairs.
 * Workspace: gsplat_hip_projection_packed_workspace_size (3/16 byte per pair,
 * plus the view-matrix partials when viewmats_grad). */
size_t gsplat_hip_projection_packed_workspace_size(int64_t B, int64_t C, int64_t N, int32_t viewmats_grad);
int gsplat_hip_projection_packed_count(const float* means, const float* covars, const float* quats,
                                       const float* scales, const float* opacities, const float* viewmats,
                                       const float* Ks, int64_t B, int64_t C, int64_t N,
                                       const gsplat_projection_params* params, int64_t* nnz_dev, void* workspace,
                                       size_t workspace_bytes, void* stream);
int gsplat_hip_projection_packed_fwd(const float* means, const float* covars, const float* quats,
                                     const float* scales, const float* opacities, const float* viewmats,
                                     const float* Ks, int64_t B, int64_t C, int64_t N,
                                     const gsplat_projection_params* params, int64_t nnz, int32_t* batch_ids,
                                     int32_t* camera_ids, int32_t* gaussian_ids, int32_t* indptr, int32_t* radii,
                                     float* means2d, float* depths, float* conics, float* compensations,
                                     const void* workspace, size_t workspace_bytes, void* stream);
int gsplat_hip_projection_packed_bwd(const float* means, const float* covars, const float* quats,
                                     const float* scales, const float* viewmats, const float* Ks, int64_t B,
                                     int64_t C, int64_t N, const gsplat_projection_params* params, int64_t nnz,
                                     const int32_t* batch_ids, const int32_t* camera_ids,
                                     const int32_t* gaussian_ids, const float* conics, const float* compensations,
                                     const float* v_means2d, const float* v_depths, const float* v_conics,
                                     const float* v_compensations, float* v_means, float* v_covars,
                                     float* v_quats, float* v_scales, float* v_viewmats, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Real spherical harmonics, degrees 0..4.
 * Replaces GSPlatSphericalHarmonics(/Backward)::eval_gpu
 * (gsplat_core/gsplat_spherical_harmonics.cpp:556-658,
 *  gsplat_core/include/gsplat_spherical_harmonics.h:35-39).
 * dirs [n,3], coeffs [n,K,3] with K >= (degree+1)^2, masks [n] (uint8/bool,
 * NULL = all on). Backward: v_dirs [n,3] (NULL = not requested),
 * v_coeffs [n,K,3].
 * ------------------------------------------------------------------------- */
int gsplat_hip_spherical_harmonics_fwd(int32_t degree, const float* dirs, const float* coeffs,
                                       const uint8_t* masks, int64_t n, int64_t K,
                                       float* colors, void* stream);
int gsplat_hip_spherical_harmonics_bwd(int32_t degree, const float* dirs, const float* coeffs,
                                       const uint8_t* masks, const float* v_colors, int64_t n,
                                       int64_t K, float* v_dirs, float* v_coeffs, void* stream);

/* Camera colours from SH with the caller's glue fused in. No counterpart
 * operator in the reference: it replaces the composition in
 * sh_colors_for_camera / camera_center_from_viewmat
 * (scanner_points_training_utils.py:1005-1034), i.e. per camera c with
 * world-to-camera matrix viewmats[c] = [R | t] (row-major 4x4) and centre
 * campos = -R^T t,
 *   n = (means - campos) / max(|means - campos|, 1e-8),
 *   colors[c] = clamp(SH_degree(n; [features_dc, features_rest]) + 0.5, 0, 1)
 * with the SH evaluated as gsplat_hip_spherical_harmonics_fwd does, and
 * without materialising the concatenated, camera-broadcast coefficients.
 * means [B,N,3], viewmats [B,C,4,4], features_dc [B,N,3], features_rest
 * [B,N,R,3] (R >= (degree+1)^2 - 1, may be NULL when R == 0),
 * colors [B,C,N,3]. The backward passes v_colors where
 * 0 < colour + 0.5 < 1 (the VJP of the reference's mx.clip, i.e. of
 * minimum(maximum(x, 0), 1): ties go to the bounds) and writes v_means, v_features_dc,
 * v_features_rest summed over the C cameras (inactive bases get 0); the view
 * matrices get no gradient.
 * radii (forward; the projection's [B,C,N,2], or NULL): a Gaussian whose
 * radii are not both positive in any camera has no tile
 * (gsplat_intersect.cpp:74-76), so a render never reads its colour and the
 * rasterizer gives it no colour gradient; given radii, the forward does not
 * read such rows and writes their colours as 0. */
int gsplat_hip_sh_camera_colors_fwd(int32_t degree, const float* means, const float* viewmats,
                                    const float* features_dc, const float* features_rest,
                                    const int32_t* radii, int64_t B, int64_t C, int64_t N, int64_t R,
                                    float* colors, void* stream);
int gsplat_hip_sh_camera_colors_bwd(int32_t degree, const float* means, const float* viewmats,
                                    const float* features_dc, const float* features_rest,
                                    const float* v_colors, int64_t B, int64_t C, int64_t N, int64_t R,
                                    float* v_means, float* v_features_dc, float* v_features_rest,
                                    void* stream);

/* The camera colours of the packed layout's pairs (no counterpart in the
 * reference; the packed render's SH colours, in place of the dense colours
 * followed by gsplat_hip_packed_rows_gather / _scatter). count_workspace is
 * the packed projection count's workspace (its rank structure: one bit per
 * pair (b, c, n) and per-word packed-row prefixes) and nnz its row count.
 * The forward writes each visible pair's colour, as
 * gsplat_hip_sh_camera_colors_fwd computes it, at the pair's packed row of
 * rows [nnz, 3], and reads only the Gaussians that some camera sees; the
 * backward reads each pair's colour cotangent at its packed row of v_rows
 * [nnz, 3] (pairs without a row: zero) and writes v_means, v_features_dc,
 * v_features_rest as gsplat_hip_sh_camera_colors_bwd does for the dense
 * cotangents with zeros at the pairs without a row. */
int gsplat_hip_sh_camera_colors_packed_fwd(int32_t degree, const float* means, const float* viewmats,
                                           const float* features_dc, const float* features_rest,
                                           const void* count_workspace, size_t count_workspace_bytes,
                                           int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R,
                                           float* rows, void* stream);
int gsplat_hip_sh_camera_colors_packed_bwd(int32_t degree, const float* means, const float* viewmats,
                                           const float* features_dc, const float* features_rest,
                                           const void* count_workspace, size_t count_workspace_bytes,
                                           const float* v_rows, int64_t nnz, int64_t B, int64_t C, int64_t N,
                                           int64_t R, float* v_means, float* v_features_dc,
                                           float* v_features_rest, void* stream);

/* ---------------------------------------------------------------------------
 * Tile intersection (dense AABB binning).
 * count + exclusive scan: replaces GSPlatIntersectTileCount::eval_gpu
 * (gsplat_core/gsplat_intersect.cpp:340-381) followed by mx::cumsum
 * (gsplat_intersect.cpp:196-211). means2d [numel,2], radii [numel,2] int32;
 * writes tiles_per_gauss [numel] and offsets [numel] (exclusive scan), and
 * the total intersection count as one int64 at *total_dev (device memory).
 * offsets may be NULL when only the counts and the total are needed (the
 * depth-presorted path below scans the counts in depth order instead); that
 * skips the scan's fix-up pass.
 * ------------------------------------------------------------------------- */
size_t gsplat_hip_isect_count_scan_workspace_size(int64_t numel);
int gsplat_hip_isect_count_scan(const float* means2d, const int32_t* radii, int64_t numel,
                                int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                int32_t* tiles_per_gauss, int32_t* offsets, int64_t* total_dev,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Exclusive scan of int32 values (out may alias in); replaces mx::cumsum
 * (inclusive=false) in gsplat_intersect_tile_offsets
 * (gsplat_core/gsplat_intersect.cpp:196-211). The int64 total is written to
 * *total_dev (device memory) when non-NULL. Partial sums must fit int32. */
size_t gsplat_hip_exclusive_scan_i32_workspace_size(int64_t n);
int gsplat_hip_exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, int64_t* total_dev,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* Replaces GSPlatIntersectTileEncode::eval_gpu (gsplat_intersect.cpp:487-538):
 * key = image << (32 + tile_bits) | tile << 32 | float_bits(depth), written
 * Gaussian-major, row-major within each Gaussian's tile rectangle, with
 * flatten_id = global (image * N + n) index. depths [numel], offsets from
 * the scan, n_isects = total. numel = I * n_per_image. */
int gsplat_hip_isect_encode(const float* means2d, const int32_t* radii, const float* depths,
                            const int32_t* offsets, int64_t I, int64_t numel,
                            int32_t tile_size, int32_t tile_width, int32_t tile_height,
                            int64_t n_isects, int64_t* isect_ids, int32_t* flatten_ids,
                            void* stream);

/* Stable ascending sort of int64 keys (non-negative) carrying int32 values;
 * replaces mx::argsort + 2x mx::take (gsplat_intersect.cpp:266-286). Only
 * the low `key_bits` bits are compared (keys must be < 2^key_bits). Inputs
 * are left unchanged. */
size_t gsplat_hip_isect_sort_workspace_size(int64_t n);
int gsplat_hip_isect_sort(const int64_t* keys_in, const int32_t* vals_in, int64_t n,
                          int32_t key_bits, int64_t* keys_out, int32_t* vals_out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Stable ascending sort of arbitrary (signed) int64 keys carrying int32
 * values, all 64 bits compared, with nothing read back to the host: the
 * digits that every key shares are found on the device from the pass
 * histograms and their passes skipped. Replaces the same mx::argsort +
 * 2x mx::take (gsplat_intersect.cpp:266-286), which takes any int64 key.
 * Workspace: gsplat_hip_isect_sort_workspace_size(n). Inputs are left
 * unchanged. */
int gsplat_hip_isect_sort_i64(const int64_t* keys_in, const int32_t* vals_in, int64_t n,
                              int64_t* keys_out, int32_t* vals_out, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Radix sort diagnostics and test hooks (no counterpart in the reference,
 * whose sort is MLX's). Every sort of this library (the standalone sort and
 * the two sorts of the intersection pipeline) runs, below 2^30 keys, one
 * onesweep kernel per 8-bit digit; a partition obtains each digit's prefix
 * by looking back over its predecessors' published counts, and a digit whose
 * predecessor stays unpublished for `spin_limit` polls recounts that prefix
 * exactly from the pass input instead (same output, no waiting).
 *  sort_debug_set: process-wide, for tests; not thread-safe with concurrent
 *    sorts. spin_limit (default 262144): 0 recounts at the first unpublished
 *    predecessor, a negative value always recounts. onesweep_max_keys
 *    (default and maximum 2^30; <= 0 restores it): sorts of at least that
 *    many keys take the reduce-then-scan path (histogram, scan, scatter per
 *    pass). Set it before querying workspace sizes: the two paths need
 *    different workspaces.
 *  sort_debug_reset: restores both defaults.
 *  sort_lookback_recounts: number of partitions (all passes, all sorts) that
 *    recounted on the current device since the library was loaded;
 *    synchronous. */
void gsplat_hip_sort_debug_set(int32_t spin_limit, int64_t onesweep_max_keys);
void gsplat_hip_sort_debug_reset(void);
int gsplat_hip_sort_lookback_recounts(uint64_t* count);

/* Test hooks of the depth-presorted intersection (no reference counterpart),
 * process-wide, not thread-safe with concurrent intersections. The sorted
 * encodes carry each entry's depth bits through the tile-key sort (rather
 * than the last pass gathering depths[flatten id]) for more than
 * carry_min_pairs pairs (default 2^21), and take every encode block's rank
 * range from one up-front search kernel (rather than searching in each block)
 * from split_min_blocks blocks on (default 65536). Negative values restore the
 * defaults. A carrying AABB sort with at least four entries per Gaussian forms
 * its first pass's keys inside that pass instead of encoding and re-reading
 * them; isect_debug_generated(0) turns that off (1, the default, on). The
 * outputs are the same either way. isect_debug_reset restores all three. */
void gsplat_hip_isect_debug_set(int64_t carry_min_pairs, int64_t split_min_blocks);
void gsplat_hip_isect_debug_generated(int32_t enable);
void gsplat_hip_isect_debug_reset(void);

/* Sorted intersections in one call: replaces the encode + sort of
 * GSPlatIntersectTile (gsplat_intersect.cpp:487-538 then :266-286) and
 * returns exactly what gsplat_hip_isect_encode followed by a stable
 * gsplat_hip_isect_sort returns -- isect_ids sorted by the 64-bit key, ties
 * in ascending flatten_id -- without sorting 64-bit keys: pairs are first
 * sorted by depth bits, encoded in that order with 32-bit (image, tile) keys,
 * and stably sorted by those. tiles_per_gauss [numel] from
 * gsplat_hip_isect_count_scan, n_isects = its total. */
size_t gsplat_hip_isect_tile_sorted_workspace_size(int64_t numel, int64_t n_isects);
int gsplat_hip_isect_tile_sorted(const float* means2d, const int32_t* radii, const float* depths,
                                 const int32_t* tiles_per_gauss, int64_t I, int64_t numel,
                                 int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                 int64_t n_isects, int64_t* isect_ids, int32_t* flatten_ids,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* The same result in two steps, so that a caller who must read the
 * intersection count back to the host can queue the first step before
 * waiting (no counterpart in the reference, whose count read-back is at
 * gsplat_intersect.cpp:155-170):
 *  depth_order: perm [numel] = pair indices stably sorted by depth bits,
 *    offsets [numel] = exclusive scan of tiles_per_gauss[perm]; needs only
 *    the counts, not their total.
 *  encode_sorted: from perm and offsets, the sorted isect_ids and
 *    flatten_ids of n_isects entries (n_isects = the counts' total). */
size_t gsplat_hip_isect_depth_order_workspace_size(int64_t numel);
int gsplat_hip_isect_depth_order(const float* depths, const int32_t* tiles_per_gauss, int64_t numel,
                                 int32_t* perm, int32_t* offsets, void* workspace,
                                 size_t workspace_bytes, void* stream);
size_t gsplat_hip_isect_encode_sorted_workspace_size(int64_t n_isects);
int gsplat_hip_isect_encode_sorted(const float* means2d, const int32_t* radii, const float* depths,
                                   const int32_t* perm, const int32_t* offsets, int64_t I, int64_t numel,
                                   int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                   int64_t n_isects, int64_t* isect_ids, int32_t* flatten_ids,
                                   void* workspace, size_t workspace_bytes, void* stream);

/* Tile-bucketed sorted intersections, the default of the C++ layer's
 * intersect_tile (sort = true, dense AABB tiles): replaces the encode + sort of
 * GSPlatIntersectTile (gsplat_intersect.cpp:487-538 then :266-286) and returns
 * what gsplat_hip_isect_encode followed by a stable gsplat_hip_isect_sort
 * returns, without a device-wide sort. Two steps around the count read-back:
 *  bucket_count: tiles_per_gauss [numel] and, at totals_dev [2] (int64,
 *    device memory), the intersection count M and the longest tile list; the
 *    count workspace (gsplat_hip_isect_bucket_count_workspace_size) then holds
 *    every tile's list start for the second step.
 *  bucket_sort: with n_isects = M and max_list = the longest list, writes the
 *    sorted isect_ids [M] and flatten_ids [M] and, when tile_offsets is not
 *    NULL, the tile offsets [I, tile_height, tile_width] (what
 *    gsplat_hip_isect_offset returns for those ids). Needs the count workspace
 *    of the same inputs and a workspace of
 *    gsplat_hip_isect_bucket_sort_workspace_size(M) bytes. Lists of up to
 *    gsplat_hip_isect_bucket_max_list() entries are sorted in LDS, longer ones
 *    split by their leading depth bits into runs sorted in LDS (or, when the
 *    split leaves a run too long, sorted in global memory).
 * Supported when gsplat_hip_isect_bucket_supported(I, tile_width, tile_height)
 * (tile grids up to about 35,000 corner points per image); otherwise use the
 * depth-presorted entry points below. */
int gsplat_hip_isect_bucket_supported(int64_t I, int32_t tile_width, int32_t tile_height);
int64_t gsplat_hip_isect_bucket_max_list(void);
size_t gsplat_hip_isect_bucket_count_workspace_size(int64_t I, int64_t numel, int32_t tile_size,
                                                    int32_t tile_width, int32_t tile_height);
int gsplat_hip_isect_bucket_count(const float* means2d, const int32_t* radii, int64_t I, int64_t numel,
                                  int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                  int32_t* tiles_per_gauss, int64_t* totals_dev, void* workspace,
                                  size_t workspace_bytes, void* stream);
size_t gsplat_hip_isect_bucket_sort_workspace_size(int64_t n_isects);
int gsplat_hip_isect_bucket_sort(const float* means2d, const int32_t* radii, const float* depths,
                                 int64_t I, int64_t numel, int32_t tile_size, int32_t tile_width,
                                 int32_t tile_height, int64_t n_isects, int64_t max_list,
                                 int64_t* isect_ids, int32_t* flatten_ids, int32_t* tile_offsets,
                                 const void* count_workspace, size_t count_workspace_bytes,
                                 void* workspace, size_t workspace_bytes, void* stream);
/* The same two steps for ellipse ("AccuTile") tiles (conics [numel,3] and
 * opacities [numel] as gsplat_hip_isect_count_scan_accutile below, which
 * the reference rejects at gsplat_intersect.cpp:123-126): the sorted lists
 * that gsplat_hip_isect_encode_accutile followed by a stable sort gives, and
 * the ellipse counts as tiles_per_gauss. Same workspaces and max_list rule;
 * supported when gsplat_hip_isect_bucket_accutile_supported(I, tile_width,
 * tile_height) (tile grids up to about 25,000 corner points per image). */
int gsplat_hip_isect_bucket_accutile_supported(int64_t I, int32_t tile_width, int32_t tile_height);
int gsplat_hip_isect_bucket_count_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                           const float* opacities, int64_t I, int64_t numel, int32_t tile_size,
                                           int32_t tile_width, int32_t tile_height, int32_t* tiles_per_gauss,
                                           int64_t* totals_dev, void* workspace, size_t workspace_bytes,
                                           void* stream);
int gsplat_hip_isect_bucket_sort_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                          const float* opacities, const float* depths, int64_t I, int64_t numel,
                                          int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                          int64_t n_isects, int64_t max_list, int64_t* isect_ids,
                                          int32_t* flatten_ids, int32_t* tile_offsets, const void* count_workspace,
                                          size_t count_workspace_bytes, void* workspace, size_t workspace_bytes,
                                          void* stream);
/* The same two steps for the packed layout (nnz rows, row r of image
 * image_ids[r]; the reference rejects packed at gsplat_intersect.cpp:115-118,
 * upstream gsplat's packed isect_tiles takes it): AABB tiles, or ellipse
 * tiles when conics and opacities are given. Flatten ids are row indices.
 * The rows must be grouped by image in ascending order, as the packed
 * projection writes them: totals_dev then holds three words, M, the longest
 * list and 0; a nonzero third word means the rows are not so grouped (or an
 * id lies outside [0, I)), and the first two words and the count workspace
 * are then not valid (use the depth-presorted packed entry points). Count
 * workspace: gsplat_hip_isect_bucket_count_packed_workspace_size(I, nnz, ...);
 * supported grids as the dense entry points (accutile_supported for ellipse
 * tiles). */
size_t gsplat_hip_isect_bucket_count_packed_workspace_size(int64_t I, int64_t nnz, int32_t tile_size,
                                                           int32_t tile_width, int32_t tile_height);
int gsplat_hip_isect_bucket_count_packed(const float* means2d, const int32_t* radii, const float* conics,
                                         const float* opacities, const int32_t* image_ids, int64_t I, int64_t nnz,
                                         int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                         int32_t* tiles_per_gauss, int64_t* totals_dev, void* workspace,
                                         size_t workspace_bytes, void* stream);
int gsplat_hip_isect_bucket_sort_packed(const float* means2d, const int32_t* radii, const float* conics,
                                        const float* opacities, const float* depths, const int32_t* image_ids,
                                        int64_t I, int64_t nnz, int32_t tile_size, int32_t tile_width,
                                        int32_t tile_height, int64_t n_isects, int64_t max_list,
                                        int64_t* isect_ids, int32_t* flatten_ids, int32_t* tile_offsets,
                                        const void* count_workspace, size_t count_workspace_bytes,
                                        void* workspace, size_t workspace_bytes, void* stream);

/* Speculative second step (no counterpart in the reference; for callers
 * that know a likely M, e.g. from the previous frame): the bucket sort of
 * any of the layouts above (ellipse tiles when conics is not NULL, packed
 * rows when packed != 0) launched before M is on the host. The kernels read
 * M from totals_dev[0] (the count step's output); capacity bounds every
 * write (isect_ids and flatten_ids hold capacity entries, the workspace
 * gsplat_hip_isect_bucket_sort_workspace_size(capacity) bytes) and max_list
 * selects the tile sort launches. The result equals the exact call's when
 * M <= capacity and gsplat_hip_isect_bucket_sort_covers(max_list, longest)
 * for the longest list read back with M; otherwise it must be discarded and
 * the exact step run. */
int gsplat_hip_isect_bucket_sort_covers(int64_t max_list_launched, int64_t longest);
int gsplat_hip_isect_bucket_sort_speculative(
    const float* means2d, const int32_t* radii, const float* conics, const float* opacities, const float* depths,
    int32_t packed, const int32_t* image_ids, int64_t I, int64_t numel, int32_t tile_size, int32_t tile_width,
    int32_t tile_height, int64_t capacity, int64_t max_list, const int64_t* totals_dev, int64_t* isect_ids,
    int32_t* flatten_ids, int32_t* tile_offsets, const void* count_workspace, size_t count_workspace_bytes,
    void* workspace, size_t workspace_bytes, void* stream);

/* Ellipse ("AccuTile") tile intersection: the use_conics / use_opacities
 * path of IntersectTileParams (gsplat_core/include/gsplat_intersect.h),
 * which the reference rejects at gsplat_intersect.cpp:123-126 and leaves to
 * upstream gsplat's IntersectTile.cu (Task_Metal.md:95-115). conics
 * [numel,3] and opacities [numel] are the rasterizer's. A Gaussian keeps the
 * tiles of its AABB rect whose pixel centres come within the ellipse
 * d^T Q d <= 2 (1.05 ln(255 o) + 1e-4); every dropped entry has
 * alpha < 1/255 at every pixel of its tile, so rendering is unchanged.
 * Opacity <= 0 gives no tiles; non-finite values, 255 o >= 3e38 and
 * conics with det <= 1e-4 a c keep the whole rect. Tiles stay row-major per
 * Gaussian. The three calls replace count_scan, encode and encode_sorted
 * (same workspaces); depth_order is shared. */
int gsplat_hip_isect_count_scan_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                         const float* opacities, int64_t numel, int32_t tile_size,
                                         int32_t tile_width, int32_t tile_height, int32_t* tiles_per_gauss,
                                         int32_t* offsets, int64_t* total_dev, void* workspace,
                                         size_t workspace_bytes, void* stream);
int gsplat_hip_isect_encode_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                     const float* opacities, const float* depths, const int32_t* offsets,
                                     int64_t I, int64_t numel, int32_t tile_size, int32_t tile_width,
                                     int32_t tile_height, int64_t n_isects, int64_t* isect_ids,
                                     int32_t* flatten_ids, void* stream);
int gsplat_hip_isect_encode_sorted_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                            const float* opacities, const float* depths, const int32_t* perm,
                                            const int32_t* offsets, int64_t I, int64_t numel, int32_t tile_size,
                                            int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                            int64_t* isect_ids, int32_t* flatten_ids, void* workspace,
                                            size_t workspace_bytes, void* stream);

/* Packed layout (IntersectTileParams.packed, rejected by the reference at
 * gsplat_intersect.cpp:115-118): nnz rows, row i in image image_ids[i]
 * (int32, in [0, I)); flatten ids are row indices. With conics and
 * opacities the ellipse tiles, else the AABB rect (both may be NULL). Counts
 * from gsplat_hip_isect_count_scan(_accutile) over the nnz rows; for the
 * sorted path, perm and offsets from gsplat_hip_isect_depth_order.
 * Workspace as gsplat_hip_isect_encode_sorted. */
int gsplat_hip_isect_encode_packed(const float* means2d, const int32_t* radii, const float* conics,
                                   const float* opacities, const int32_t* image_ids, const float* depths,
                                   const int32_t* offsets, int64_t I, int64_t nnz, int32_t tile_size,
                                   int32_t tile_width, int32_t tile_height, int64_t n_isects, int64_t* isect_ids,
                                   int32_t* flatten_ids, void* stream);
int gsplat_hip_isect_encode_sorted_packed(const float* means2d, const int32_t* radii, const float* conics,
                                          const float* opacities, const int32_t* image_ids, const float* depths,
                                          const int32_t* perm, const int32_t* offsets, int64_t I, int64_t nnz,
                                          int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                          int64_t n_isects, int64_t* isect_ids, int32_t* flatten_ids,
                                          void* workspace, size_t workspace_bytes, void* stream);

/* Replaces GSPlatIntersectOffset::eval_gpu (gsplat_intersect.cpp:643-681):
 * offsets [I, tile_height, tile_width] = lower_bound of (image << tile_bits |
 * tile) over the sorted isect_ids >> 32. */
int gsplat_hip_isect_offset(const int64_t* isect_ids, int64_t n_isects, int32_t I,
                            int32_t tile_width, int32_t tile_height, int32_t* offsets,
                            void* stream);

/* ---------------------------------------------------------------------------
 * Rasterization to pixels (front-to-back alpha compositing).
 * Replaces GSPlatRasterizeToPixels3DGS(/Backward)::eval_gpu
 * (gsplat_core/gsplat_rasterize.cpp:571-738,
 *  gsplat_core/include/gsplat_rasterize.h:67-71).
 * means2d [I,N,2], conics [I,N,3], colors [I,N,channels], opacities [I,N],
 * backgrounds [I,channels] (NULL = black), masks [I,th,tw] (NULL = all on),
 * tile_offsets [I,th,tw], flatten_ids [n_isects].
 * Forward outputs: render_colors [I,H,W,channels], render_alphas [I,H,W],
 * last_ids [I,H,W]. Backward outputs (accumulated over all pixels):
 * v_means2d_abs (NULL unless absgrad), v_means2d, v_conics, v_colors,
 * v_opacities, v_backgrounds (NULL unless backgrounds). The backward's
 * v_render_alphas may be NULL, meaning zeros (losses on the colours only).
 * ------------------------------------------------------------------------- */
int gsplat_hip_rasterize_fwd(const float* means2d, const float* conics, const float* colors,
                             const float* opacities, const float* backgrounds,
                             const uint8_t* masks, const int32_t* tile_offsets,
                             const int32_t* flatten_ids, int64_t I, int64_t N, int32_t channels,
                             int32_t image_width, int32_t image_height, int32_t tile_size,
                             int32_t tile_width, int32_t tile_height, int64_t n_isects,
                             float* render_colors, float* render_alphas, int32_t* last_ids,
                             void* stream);
/* Measurement, no counterpart in the reference: E_f, the (pixel, list entry)
 * evaluations of the reference's forward loop (gsplat_rasterize.cpp:291-368:
 * every entry of a pixel's tile list up to and including the one that takes
 * its transmittance to 1e-4), per tile into tile_evals [I, tile_height,
 * tile_width] (int64). Inputs as gsplat_hip_rasterize_fwd (G Gaussian rows;
 * colours are not needed). The unit of work the rasterizer's roofline is
 * priced on. */
int gsplat_hip_rasterize_count_evals(const float* means2d, const float* conics, const float* opacities,
                                     const uint8_t* masks, const int32_t* tile_offsets,
                                     const int32_t* flatten_ids, int64_t I, int64_t G, int32_t image_width,
                                     int32_t image_height, int32_t tile_size, int32_t tile_width,
                                     int32_t tile_height, int64_t n_isects, int64_t* tile_evals, void* stream);
int gsplat_hip_rasterize_bwd(const float* means2d, const float* conics, const float* colors,
                             const float* opacities, const float* backgrounds,
                             const uint8_t* masks, const int32_t* tile_offsets,
                             const int32_t* flatten_ids, int64_t I, int64_t N, int32_t channels,
                             int32_t image_width, int32_t image_height, int32_t tile_size,
                             int32_t tile_width, int32_t tile_height, int64_t n_isects,
                             const float* render_alphas, const int32_t* last_ids,
                             const float* v_render_colors, const float* v_render_alphas,
                             float* v_means2d_abs, float* v_means2d, float* v_conics,
                             float* v_colors, float* v_opacities, float* v_backgrounds,
                             void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of device workspace rasterize_bwd needs for I images of
 * tile_width x tile_height tiles and `channels` colour channels (its
 * heavy-first tile schedule: one cost and one order entry per tile; and one
 * background-gradient partial per tile and channel). No counterpart in the
 * reference, whose CPU backward allocates nothing of the kind. */
size_t gsplat_hip_rasterize_bwd_workspace_size(int64_t I, int32_t channels, int32_t tile_width,
                                               int32_t tile_height);

/* Allocation-free variant of gsplat_hip_rasterize_bwd. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and outputs as gsplat_hip_rasterize_bwd without the
 * workspace: the tile schedule and background partials live in a static
 * device array of the library, 8 MiB per GPU, held until the process ends
 * (gsplat_hip_rasterize_bwd_noalloc_max_scratch() returns the size). Sizes
 * whose schedule needs more (about I * tiles * (8 + 4 * channels) bytes,
 * e.g. more than 400k tiles at 3 channels) are rejected with
 * GSPLAT_ERR_INVALID_ARGUMENT. It calls no hipMalloc / hipFree and no
 * allocating library routine (with kernel timing off); its first call on a
 * device looks up that device's array address once. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (several streams
 * or host threads at once) race and must be serialized by the caller. */
size_t gsplat_hip_rasterize_bwd_noalloc_max_scratch(void);
int gsplat_hip_rasterize_bwd_noalloc(const float* means2d, const float* conics, const float* colors,
                                     const float* opacities, const float* backgrounds,
                                     const uint8_t* masks, const int32_t* tile_offsets,
                                     const int32_t* flatten_ids, int64_t I, int64_t N, int32_t channels,
                                     int32_t image_width, int32_t image_height, int32_t tile_size,
                                     int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                     const float* render_alphas, const int32_t* last_ids,
                                     const float* v_render_colors, const float* v_render_alphas,
                                     float* v_means2d_abs, float* v_means2d, float* v_conics,
                                     float* v_colors, float* v_opacities, float* v_backgrounds,
                                     void* stream);

/* Packed layout (RasterizeToPixels3DGSParams.packed, rejected by the
 * reference at gsplat_rasterize.cpp:48-51): the Gaussian arrays have nnz rows
 * (means2d [nnz,2], conics [nnz,3], colors [nnz,channels], opacities [nnz])
 * and flatten_ids index them; images, backgrounds and masks are as dense
 * ([I, ...], I from tile_offsets). Gradients have nnz rows. Otherwise as the
 * dense entry points (same workspace). */
int gsplat_hip_rasterize_fwd_packed(const float* means2d, const float* conics, const float* colors,
                                    const float* opacities, const float* backgrounds, const uint8_t* masks,
                                    const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I,
                                    int64_t nnz, int32_t channels, int32_t image_width, int32_t image_height,
                                    int32_t tile_size, int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                    float* render_colors, float* render_alphas, int32_t* last_ids, void* stream);
int gsplat_hip_rasterize_bwd_packed(const float* means2d, const float* conics, const float* colors,
                                    const float* opacities, const float* backgrounds, const uint8_t* masks,
                                    const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I,
                                    int64_t nnz, int32_t channels, int32_t image_width, int32_t image_height,
                                    int32_t tile_size, int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                    const float* render_alphas, const int32_t* last_ids,
                                    const float* v_render_colors, const float* v_render_alphas,
                                    float* v_means2d_abs, float* v_means2d, float* v_conics, float* v_colors,
                                    float* v_opacities, float* v_backgrounds, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* Rasterize to indices: upstream gsplat's rasterize_to_indices_in_range
 * (note/gsplat_cuda_source_map.md:494-545; the reference's planned
 * rasterize_to_indices_3dgs_forward). For each pixel, starting from
 * transmittances[pixel] (NULL: 1), the entries of its tile's list at
 * positions [range_start, range_end) that the forward would composite (alpha
 * test passed, in list order, until the transmittance would fall to 1e-4).
 * Gaussian arrays have n_rows rows (I * N dense, nnz packed); masks are not
 * taken. count: per-pixel counts scanned into starts [I*H*W] (exclusive) and
 * the total at *total_dev (device int64; the caller reads it back); write:
 * out_gauss_ids [n_out] (flatten ids) and out_indices [n_out] (image * H * W +
 * y * W + x), pixel-major, list order within a pixel. */
size_t gsplat_hip_rasterize_to_indices_workspace_size(int64_t I, int32_t image_width, int32_t image_height);
int gsplat_hip_rasterize_to_indices_count(int64_t range_start, int64_t range_end, const float* transmittances,
                                          const float* means2d, const float* conics, const float* opacities,
                                          const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I,
                                          int64_t n_rows, int32_t image_width, int32_t image_height,
                                          int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                          int64_t n_isects, int32_t* starts, int64_t* total_dev, void* workspace,
                                          size_t workspace_bytes, void* stream);
int gsplat_hip_rasterize_to_indices_write(int64_t range_start, int64_t range_end, const float* transmittances,
                                          const float* means2d, const float* conics, const float* opacities,
                                          const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I,
                                          int64_t n_rows, int32_t image_width, int32_t image_height,
                                          int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                          int64_t n_isects, const int32_t* starts, int64_t n_out,
                                          int32_t* out_gauss_ids, int64_t* out_indices, void* stream);

/* ---------------------------------------------------------------------------
 * Training-step glue around the chain, one kernel per direction. No
 * counterpart operator in the reference: these replace the framework
 * elementwise composition at its call sites.
 * Parameter activations (scanner_points_training_utils.py:39-41 and the
 * model properties at :306-316), n Gaussians:
 *   quats_out [n,4] = quats / max(|quats|, 1e-8), scales_out [n,3] =
 *   exp(log_scales), opacities_out [n] = sigmoid(opacity_logits).
 * Any input group may be NULL (skipped). The backward writes v_quats,
 * v_log_scales, v_logits (each may be NULL); a NULL cotangent counts as zero.
 * It reads the raw quats and the forward's scales and opacities. */
int gsplat_hip_gaussian_activations_fwd(const float* quats, const float* log_scales,
                                        const float* opacity_logits, int64_t n, float* quats_out,
                                        float* scales_out, float* opacities_out, void* stream);
int gsplat_hip_gaussian_activations_bwd(const float* quats, const float* scales, const float* opacities,
                                        const float* v_quats_out, const float* v_scales,
                                        const float* v_opacities, int64_t n, float* v_quats,
                                        float* v_log_scales, float* v_logits, void* stream);

/* Activated projection: the activations above fused into the fused EWA
 * projection (gsplat_hip_projection_fwd / _bwd, pinhole backward only), for
 * callers whose model stores raw parameters. quats [B,N,4] are raw
 * quaternions, log_scales [B,N,3] and opacity_logits [B,N] the logarithms and
 * logits; use_covars must be 0. Outputs as gsplat_hip_projection_fwd plus
 * opacities [B,N] = sigmoid(opacity_logits) when non-NULL (opacity_logits
 * NULL: no opacities; use_opacities then must be 0). The results equal
 * gsplat_hip_gaussian_activations_fwd followed by gsplat_hip_projection_fwd
 * bit for bit. The backward takes the projection cotangents plus
 * v_opacities [B,N] (NULL: zeros) and writes v_means, v_quats and
 * v_log_scales (raw-parameter gradients), v_opacity_logits [B,N] (may be
 * NULL) and v_viewmats as gsplat_hip_projection_bwd (same workspace). */
int gsplat_hip_activated_projection_fwd(const float* means, const float* quats,
                                        const float* log_scales, const float* opacity_logits,
                                        const float* viewmats, const float* Ks, int64_t B,
                                        int64_t C, int64_t N, const gsplat_projection_params* params,
                                        int32_t* radii, float* means2d, float* depths, float* conics,
                                        float* compensations, float* opacities, void* stream);
int gsplat_hip_activated_projection_bwd(const float* means, const float* quats,
                                        const float* log_scales, const float* opacity_logits,
                                        const float* viewmats, const float* Ks, int64_t B,
                                        int64_t C, int64_t N, const gsplat_projection_params* params,
                                        const int32_t* radii, const float* conics,
                                        const float* compensations, const float* v_means2d,
                                        const float* v_depths, const float* v_conics,
                                        const float* v_compensations, const float* v_opacities,
                                        float* v_means, float* v_quats, float* v_log_scales,
                                        float* v_opacity_logits, float* v_viewmats, void* workspace,
                                        size_t workspace_bytes, void* stream);

/* Activated packed projection (no reference counterpart): the activations
 * fused into the packed projection (gsplat_hip_projection_packed_count /
 * _fwd / _bwd), for the packed training step of a model with raw
 * parameters. Inputs as gsplat_hip_activated_projection_fwd; the count and
 * forward take the workspace of gsplat_hip_projection_packed_workspace_size(
 * B, C, N, 0) and give the same rows as gsplat_hip_gaussian_activations_fwd
 * followed by the packed projection, bit for bit, plus opacities [nnz] (when
 * non-NULL; needs opacity_logits), each visible pair's sigmoid opacity. With
 * nnz_dev (the count's device total) the forward may run before the count is
 * on the host: nnz is then the outputs' capacity (rows past it are not
 * written; the result is whole when the count is at most nnz) and indptr
 * ends with the device total. The
 * caller keeps the count's workspace for the backward (count_workspace): it
 * holds the rank structure that maps a pair to its row, so the backward takes
 * no ids. The backward's cotangents are per row, v_opacities [nnz] included
 * (NULL: zeros; it is summed over a Gaussian's pairs in camera order), and it
 * writes the raw parameters' gradients as gsplat_hip_activated_projection_bwd,
 * with its own workspace of gsplat_hip_projection_packed_workspace_size(B, C,
 * N, v_viewmats != NULL), plus v_viewspace [B, C, N, 2] when non-NULL: each
 * pair's v_means2d row, zeros for pairs without a row (the gradient of a
 * dense viewspace proxy of the means2d). */
int gsplat_hip_activated_projection_packed_count(const float* means, const float* quats,
                                                 const float* log_scales, const float* opacity_logits,
                                                 const float* viewmats, const float* Ks, int64_t B,
                                                 int64_t C, int64_t N, const gsplat_projection_params* params,
                                                 int64_t* nnz_dev, void* workspace, size_t workspace_bytes,
                                                 void* stream);
int gsplat_hip_activated_projection_packed_fwd(const float* means, const float* quats,
                                               const float* log_scales, const float* opacity_logits,
                                               const float* viewmats, const float* Ks, int64_t B, int64_t C,
                                               int64_t N, const gsplat_projection_params* params, int64_t nnz,
                                               const int64_t* nnz_dev, int32_t* batch_ids, int32_t* camera_ids,
                                               int32_t* gaussian_ids, int32_t* indptr, int32_t* radii,
                                               float* means2d, float* depths, float* conics, float* compensations,
                                               float* opacities, const void* workspace, size_t workspace_bytes,
                                               void* stream);
int gsplat_hip_activated_projection_packed_bwd(const float* means, const float* quats,
                                               const float* log_scales, const float* opacity_logits,
                                               const float* viewmats, const float* Ks, int64_t B, int64_t C,
                                               int64_t N, const gsplat_projection_params* params, int64_t nnz,
                                               const void* count_workspace, size_t count_workspace_bytes,
                                               const float* conics, const float* compensations,
                                               const float* v_means2d, const float* v_depths,
                                               const float* v_conics, const float* v_compensations,
                                               const float* v_opacities, float* v_means, float* v_quats,
                                               float* v_log_scales, float* v_opacity_logits, float* v_viewmats,
                                               float* v_viewspace, void* workspace, size_t workspace_bytes,
                                               void* stream);

/* Packed rows <-> dense slots (no reference counterpart; the packed
 * training step's per-row colours): gather rows [nnz, K] = dense [B, C, N, K]
 * at each row's (batch, camera, Gaussian) (batch_ids may be NULL with B = 1;
 * ids outside the grid give zeros); scatter, its adjoint, writes every dense
 * slot: the row's values where the pair has a row (the count pass's rank
 * structure, as the activated packed backward reads it), zeros elsewhere. */
int gsplat_hip_packed_rows_gather(const float* dense, const int32_t* batch_ids, const int32_t* camera_ids,
                                  const int32_t* gaussian_ids, int64_t nnz, int64_t B, int64_t C, int64_t N,
                                  int32_t K, float* rows, void* stream);
int gsplat_hip_packed_rows_scatter(const float* rows, const void* count_workspace, size_t count_workspace_bytes,
                                   int64_t nnz, int64_t B, int64_t C, int64_t N, int32_t K, float* dense,
                                   void* stream);

/* Image L1 term mean(|a - b|) over n values into the device scalar *loss
 * (nn.losses.l1_loss in image_loss_components,
 * scanner_points_training_utils.py:1147-1160). The backward reads the device scalar cotangent
 * *grad and writes v_a = grad / n * sign(a - b) and v_b = -v_a (either may be
 * NULL). */
size_t gsplat_hip_l1_loss_workspace_size(int64_t n);
int gsplat_hip_l1_loss_fwd(const float* a, const float* b, int64_t n, float* loss, void* workspace,
                           size_t workspace_bytes, void* stream);
int gsplat_hip_l1_loss_bwd(const float* a, const float* b, int64_t n, const float* grad, float* v_a,
                           float* v_b, void* stream);

/* Image loss of image_loss_components with loss_mode "l1_dssim"
 * (scanner_points_training_utils.py:1123-1172: local_average, ssim_index and
 * the L1 term) for image and target [B, H, W, C] float32 (NHWC): out[0] =
 * mean|image - target|, out[1] = ssim_index(image, target, window) -- the mean
 * over the [B, Ho, Wo, C] map (Ho = H + 2 (window / 2) - window + 1, Wo
 * likewise) of the SSIM of window x window box means with zero padding, c1 =
 * 0.01^2, c2 = 0.03^2 and the denominator clamped at 1e-12. maps (NULL: not
 * written) receives gsplat_hip_image_loss_map_size() * 3 floats, three planes
 * of per-window derivatives for the backward. Requires (window - 1) * C <= 768.
 * An empty image gives NaN for both means. The backward writes
 * v_image = g_l1 / n * sign(image - target) + g_ssim * d ssim / d image from
 * the device scalar cotangents g_l1 and g_ssim (either may be NULL: zero;
 * g_ssim needs the forward's maps); the target gets no gradient. */
int64_t gsplat_hip_image_loss_map_size(int64_t B, int64_t H, int64_t W, int64_t C, int window);
size_t gsplat_hip_image_loss_workspace_size(int64_t B, int64_t H, int64_t W, int64_t C, int window);
int gsplat_hip_image_loss_fwd(const float* image, const float* target, int64_t B, int64_t H, int64_t W,
                              int64_t C, int window, float* out, float* maps, void* workspace,
                              size_t workspace_bytes, void* stream);
int gsplat_hip_image_loss_bwd(const float* image, const float* target, const float* maps, int64_t B,
                              int64_t H, int64_t W, int64_t C, int window, const float* g_l1,
                              const float* g_ssim, float* v_image, void* stream);

/* Selective Adam: upstream gsplat's fused selective_adam_update
 * (note/gsplat_cuda_source_map.md:575-577), the optimizer step after the
 * VJPs. In place over n rows of D values (param, grad, exp_avg, exp_avg_sq
 * [n, D]); rows with valid[row] == 0 are left unchanged (valid NULL: all
 * rows). m = b1 m + (1 - b1) g; v = b2 v + (1 - b2) g^2;
 * param -= (lr / bias_correction1) m / (sqrt(v) / bias_correction2_sqrt + eps)
 * -- torch.optim.Adam's step with bias_correction1 = 1 - b1^t and
 * bias_correction2_sqrt = sqrt(1 - b2^t); 1 and 1 give upstream's form. The
 * scalars are double: 1 - b1, 1 - b2 and lr / bias_correction1 are formed in
 * double and rounded once, as torch forms them from Python floats. */
int gsplat_hip_selective_adam(float* param, const float* grad, float* exp_avg, float* exp_avg_sq,
                              const uint8_t* valid, int64_t n, int64_t D, double lr, double b1, double b2,
                              double eps, double bias_correction1, double bias_correction2_sqrt, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* GSPLAT_HIP_H_ */
