// Spherical harmonics operator layer: validation and shapes follow
// gsplat_core/gsplat_spherical_harmonics.cpp:33-110, 429-464 of the
// reference; compute is the HIP C-ABI.
#include "gsplat_spherical_harmonics.h"

#include "core_util.h"

namespace gsplat_core {
namespace {
using namespace detail;

void validate_common(const char* op, int degree, const array& dirs, const array& coeffs, const array& masks,
                     bool use_masks) {
  if (degree < 0 || degree > 4) throw std::runtime_error(std::string(op) + " supports degree 0..4.");
  if (dirs.dim() < 1 || dirs.size(-1) != 3) throw std::runtime_error("dirs must have shape [..., 3].");
  if (coeffs.dim() < 2 || coeffs.size(-1) != 3) throw std::runtime_error("coeffs must have shape [..., K, 3].");
  const int64_t k = coeffs.size(-2);
  if (k < (degree + 1) * (degree + 1))
    throw std::runtime_error("coeffs has fewer SH bases than degrees_to_use requires.");
  if (coeffs.numel() / (k * 3) != dirs.numel() / 3)
    throw std::runtime_error("dirs and coeffs prefix dimensions must have the same size.");
  if (use_masks && masks.numel() != dirs.numel() / 3)
    throw std::runtime_error("masks must have shape matching dirs prefix dims.");
}

}  // namespace

array gsplat_spherical_harmonics_forward(const SphericalHarmonicsInput& input) {
  if (input.dirs.scalar_type() != at::kFloat || input.coeffs.scalar_type() != at::kFloat)
    throw std::runtime_error("spherical_harmonics_forward currently supports float32 dirs and coeffs.");
  validate_common("spherical_harmonics_forward", input.degrees_to_use, input.dirs, input.coeffs, input.masks,
                  input.use_masks);
  require_device(input.dirs, "dirs");
  require_device(input.coeffs, "coeffs");
  if (input.use_masks) require_device(input.masks, "masks");
  const c10::DeviceGuard guard(input.dirs.device());
  const array dirs = contig(input.dirs);
  const array coeffs = contig(input.coeffs);
  const array masks = input.use_masks ? mask_u8(input.masks) : array();
  array colors = at::empty(dirs.sizes(), f32_like(dirs));
  check(gsplat_hip_spherical_harmonics_fwd(input.degrees_to_use, dirs.data_ptr<float>(), coeffs.data_ptr<float>(),
                                           input.use_masks ? masks.data_ptr<uint8_t>() : nullptr, dirs.numel() / 3,
                                           coeffs.size(-2), colors.data_ptr<float>(), stream_for(input.s, dirs)));
  return colors;
}

std::vector<array> gsplat_spherical_harmonics_backward(const SphericalHarmonicsBackwardInput& input) {
  if (input.dirs.scalar_type() != at::kFloat || input.coeffs.scalar_type() != at::kFloat ||
      input.v_colors.scalar_type() != at::kFloat)
    throw std::runtime_error("spherical_harmonics_backward currently supports float32 arrays.");
  if (input.dirs.dim() < 1 || input.dirs.size(-1) != 3) throw std::runtime_error("dirs must have shape [..., 3].");
  if (input.v_colors.sizes() != input.dirs.sizes())
    throw std::runtime_error("v_colors must have the same shape as dirs.");
  validate_common("spherical_harmonics_backward", input.degrees_to_use, input.dirs, input.coeffs, input.masks,
                  input.use_masks);
  require_device(input.dirs, "dirs");
  require_device(input.coeffs, "coeffs");
  require_device(input.v_colors, "v_colors");
  if (input.use_masks) require_device(input.masks, "masks");
  const c10::DeviceGuard guard(input.dirs.device());
  const array dirs = contig(input.dirs);
  const array coeffs = contig(input.coeffs);
  const array v_colors = contig(input.v_colors);
  const array masks = input.use_masks ? mask_u8(input.masks) : array();
  array v_dirs = input.compute_v_dirs ? at::empty(dirs.sizes(), f32_like(dirs)) : at::empty({0}, f32_like(dirs));
  array v_coeffs = at::empty(coeffs.sizes(), f32_like(dirs));
  check(gsplat_hip_spherical_harmonics_bwd(
      input.degrees_to_use, dirs.data_ptr<float>(), coeffs.data_ptr<float>(),
      input.use_masks ? masks.data_ptr<uint8_t>() : nullptr, v_colors.data_ptr<float>(), dirs.numel() / 3,
      coeffs.size(-2), input.compute_v_dirs ? v_dirs.data_ptr<float>() : nullptr, v_coeffs.data_ptr<float>(),
      stream_for(input.s, dirs)));
  return {v_dirs, v_coeffs};
}

}  // namespace gsplat_core
