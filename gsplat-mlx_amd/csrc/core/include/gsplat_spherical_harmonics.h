// Spherical harmonics operator API; mirrors
// gsplat_core/include/gsplat_spherical_harmonics.h:10-39 of the reference.
#pragma once

#include "gsplat_common.h"

namespace gsplat_core {

struct SphericalHarmonicsInput {
  int degrees_to_use;
  array dirs;
  array coeffs;
  array masks;
  StreamOrDevice s;
  bool use_masks;
};

struct SphericalHarmonicsBackwardInput {
  int degrees_to_use;
  array dirs;
  array coeffs;
  array masks;
  array v_colors;
  StreamOrDevice s;
  bool use_masks;
  bool compute_v_dirs;
};

enum SphericalHarmonicsBackwardOutputIndex {
  kSHVDirs = 0,
  kSHVCoeffs = 1,
};

array gsplat_spherical_harmonics_forward(const SphericalHarmonicsInput& input);

std::vector<array> gsplat_spherical_harmonics_backward(const SphericalHarmonicsBackwardInput& input);

// Caller-side composition fused into one kernel per direction (no reference
// counterpart as an operator; it is the glue of
// scanner_points_training_utils.py:1005-1034): colors [B, C, N, 3] =
// clamp(SH(normalize(means - campos[c]); [dc, rest]) + 0.5, 0, 1) with
// campos[c] = -R^T t of viewmats[c] = [R | t], for means [B, N, 3], viewmats
// [B, C, 4, 4], features_dc [B, N, 3], features_rest [B, N, R, 3]
// (R >= (degree + 1)^2 - 1). radii (optional: undefined or empty for none):
// the projection's [B, C, N, 2]; rows whose radii are not both positive in
// any camera (no tile, so no render reads them) are then skipped and get
// colour 0.
array gsplat_sh_camera_colors_forward(int degree, const array& means, const array& viewmats, const array& features_dc,
                                      const array& features_rest, const array& radii = array(),
                                      StreamOrDevice s = {});

// Gradients {v_means, v_features_dc, v_features_rest} of the above, summed
// over cameras (viewmats get none).
std::vector<array> gsplat_sh_camera_colors_backward(int degree, const array& means, const array& viewmats,
                                                    const array& features_dc, const array& features_rest,
                                                    const array& v_colors, StreamOrDevice s = {});

// The camera colours of the packed layout's pairs: rank is the packed
// projection's count workspace (its "rank" output: one bit per (b, c, n)
// pair and per-word packed-row prefixes) and nnz its row count. The forward
// returns [nnz, 3], each visible pair's colour as above at its packed row;
// the backward takes the rows' cotangents [nnz, 3] and returns {v_means,
// v_features_dc, v_features_rest} as above for the dense cotangents with
// zeros at the pairs without a row.
array gsplat_sh_camera_colors_packed_forward(int degree, const array& means, const array& viewmats,
                                             const array& features_dc, const array& features_rest,
                                             const array& rank, int64_t nnz, StreamOrDevice s = {});
std::vector<array> gsplat_sh_camera_colors_packed_backward(int degree, const array& means, const array& viewmats,
                                                           const array& features_dc, const array& features_rest,
                                                           const array& rank, const array& v_rows,
                                                           StreamOrDevice s = {});

}  // namespace gsplat_core
