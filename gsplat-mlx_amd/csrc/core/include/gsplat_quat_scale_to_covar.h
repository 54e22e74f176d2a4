// quat_scale_to_covar_preci operator API; mirrors
// gsplat_core/include/gsplat_quat_scale_to_covar.h:12-46 of the reference.
#pragma once

#include "gsplat_common.h"

namespace gsplat_core {

struct QuatScaleToCovarPreciInput {
  array quats;
  array scales;
  StreamOrDevice s;
  bool compute_covar;
  bool compute_preci;
  bool triu;
};

struct QuatScaleToCovarPreciBackwardInput {
  array quats;
  array scales;
  array v_covars;
  array v_precis;
  StreamOrDevice s;
  bool triu;
  bool use_v_covars;
  bool use_v_precis;
};

enum QuatScaleToCovarPreciOutputIndex {
  kCovars = 0,
  kPrecis = 1,
};

enum QuatScaleToCovarPreciBackwardOutputIndex {
  kVQuats = 0,
  kVScales = 1,
};

std::vector<array> gsplat_quat_scale_to_covar_preci_forward(const QuatScaleToCovarPreciInput& input);

std::vector<array> gsplat_quat_scale_to_covar_preci_backward(const QuatScaleToCovarPreciBackwardInput& input);

}  // namespace gsplat_core
