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

}  // namespace gsplat_core
