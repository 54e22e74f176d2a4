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

}  // namespace gsplat_core
