// quat_scale_to_covar_preci operator layer: validation and shapes follow
// gsplat_core/gsplat_quat_scale_to_covar.cpp:35-101, 335-372 of the
// reference; compute is the HIP C-ABI.
#include "gsplat_quat_scale_to_covar.h"

#include "core_util.h"

namespace gsplat_core {
namespace {
using namespace detail;

std::vector<int64_t> output_shape(const array& quats, bool triu) {
  std::vector<int64_t> shape(quats.sizes().begin(), quats.sizes().end() - 1);
  if (triu) {
    shape.push_back(6);
  } else {
    shape.push_back(3);
    shape.push_back(3);
  }
  return shape;
}

void validate_common(const array& quats, const array& scales) {
  if (quats.dim() < 1 || quats.size(-1) != 4) throw std::runtime_error("quats must have shape [..., 4].");
  if (scales.dim() < 1 || scales.size(-1) != 3) throw std::runtime_error("scales must have shape [..., 3].");
  if (quats.numel() / 4 != scales.numel() / 3)
    throw std::runtime_error("quats and scales prefix dimensions must have the same size.");
}

}  // namespace

std::vector<array> gsplat_quat_scale_to_covar_preci_forward(const QuatScaleToCovarPreciInput& input) {
  if (input.quats.scalar_type() != at::kFloat || input.scales.scalar_type() != at::kFloat)
    throw std::runtime_error("quat_scale_to_covar_preci_forward currently supports float32 inputs.");
  validate_common(input.quats, input.scales);
  require_device(input.quats, "quats");
  require_device(input.scales, "scales");
  const c10::DeviceGuard guard(input.quats.device());
  const array q = contig(input.quats);
  const array s = contig(input.scales);
  const auto shape = output_shape(q, input.triu);
  array covars = input.compute_covar ? at::empty(shape, f32_like(q)) : at::empty({0}, f32_like(q));
  array precis = input.compute_preci ? at::empty(shape, f32_like(q)) : at::empty({0}, f32_like(q));
  const int64_t n = q.numel() / 4;
  check(gsplat_hip_quat_scale_to_covar_preci_fwd(q.data_ptr<float>(), s.data_ptr<float>(), n, input.compute_covar,
                                                 input.compute_preci, input.triu,
                                                 input.compute_covar ? covars.data_ptr<float>() : nullptr,
                                                 input.compute_preci ? precis.data_ptr<float>() : nullptr,
                                                 stream_for(input.s, q)));
  return {covars, precis};
}

std::vector<array> gsplat_quat_scale_to_covar_preci_backward(const QuatScaleToCovarPreciBackwardInput& input) {
  if (input.quats.scalar_type() != at::kFloat || input.scales.scalar_type() != at::kFloat)
    throw std::runtime_error("quat_scale_to_covar_preci_backward currently supports float32 inputs.");
  if (input.use_v_covars && input.v_covars.scalar_type() != at::kFloat)
    throw std::runtime_error("v_covars must be float32.");
  if (input.use_v_precis && input.v_precis.scalar_type() != at::kFloat)
    throw std::runtime_error("v_precis must be float32.");
  validate_common(input.quats, input.scales);
  const auto expected = output_shape(input.quats, input.triu);
  if (input.use_v_covars && input.v_covars.sizes().vec() != expected)
    throw std::runtime_error("v_covars shape does not match triu output shape.");
  if (input.use_v_precis && input.v_precis.sizes().vec() != expected)
    throw std::runtime_error("v_precis shape does not match triu output shape.");
  require_device(input.quats, "quats");
  require_device(input.scales, "scales");
  if (input.use_v_covars) require_device(input.v_covars, "v_covars");
  if (input.use_v_precis) require_device(input.v_precis, "v_precis");
  const c10::DeviceGuard guard(input.quats.device());
  const array q = contig(input.quats);
  const array s = contig(input.scales);
  const array vc = input.use_v_covars ? contig(input.v_covars) : array();
  const array vp = input.use_v_precis ? contig(input.v_precis) : array();
  array v_quats = at::empty(q.sizes(), f32_like(q));
  array v_scales = at::empty(s.sizes(), f32_like(q));
  check(gsplat_hip_quat_scale_to_covar_preci_bwd(q.data_ptr<float>(), s.data_ptr<float>(),
                                                 input.use_v_covars ? vc.data_ptr<float>() : nullptr,
                                                 input.use_v_precis ? vp.data_ptr<float>() : nullptr,
                                                 q.numel() / 4, input.triu, v_quats.data_ptr<float>(),
                                                 v_scales.data_ptr<float>(), stream_for(input.s, q)));
  return {v_quats, v_scales};
}

}  // namespace gsplat_core
