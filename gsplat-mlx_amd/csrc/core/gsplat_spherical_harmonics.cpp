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

struct CamDims {
  int64_t B, C, N, R;
};

CamDims validate_camera(const char* op, int degree, const array& means, const array& viewmats, const array& dc,
                        const array& rest) {
  const std::string o(op);
  if (degree < 0 || degree > 4) throw std::runtime_error(o + " supports degree 0..4.");
  if (means.dim() < 2 || means.size(-1) != 3) throw std::runtime_error("means must have shape [..., N, 3].");
  if (viewmats.dim() < 3 || viewmats.size(-1) != 4 || viewmats.size(-2) != 4)
    throw std::runtime_error("viewmats must have shape [..., C, 4, 4].");
  if (dc.sizes() != means.sizes()) throw std::runtime_error("features_dc must have the shape of means.");
  if (rest.dim() != means.dim() + 1 || rest.size(-1) != 3)
    throw std::runtime_error("features_rest must have shape [..., N, R, 3].");
  for (const array* a : {&means, &viewmats, &dc, &rest})
    if (a->scalar_type() != at::kFloat) throw std::runtime_error(o + " supports float32 arrays only.");
  CamDims d;
  d.N = means.size(-2);
  d.B = d.N > 0 ? means.numel() / (d.N * 3) : 0;
  d.C = viewmats.size(-3);
  d.R = rest.size(-2);
  if (viewmats.numel() != d.B * d.C * 16) throw std::runtime_error("viewmats batch dimensions must match means.");
  if (rest.numel() != d.B * d.N * d.R * 3) throw std::runtime_error("features_rest batch dimensions must match means.");
  if (d.R < (degree + 1) * (degree + 1) - 1)
    throw std::runtime_error("features_rest has fewer SH bases than degrees_to_use requires.");
  require_device(means, "means");
  require_device(viewmats, "viewmats");
  require_device(dc, "features_dc");
  require_device(rest, "features_rest");
  return d;
}

// The optional radii of the camera colour functions: [..., C, N, 2] int32 on
// the means' device, or none (undefined or empty).
const int32_t* camera_radii(const array& radii, const CamDims& d, const array& means, array& keep, const char* what) {
  if (!radii.defined() || radii.numel() == 0) return nullptr;
  const std::string o(what);
  if (radii.scalar_type() != at::kInt) throw std::runtime_error(o + ": radii must be int32.");
  if (radii.numel() != d.B * d.C * d.N * 2 || radii.size(-1) != 2)
    throw std::runtime_error(o + ": radii must have shape [..., C, N, 2].");
  if (radii.device() != means.device()) throw std::runtime_error(o + ": radii must be on the means' device.");
  keep = contig(radii);
  return keep.data_ptr<int32_t>();
}

}  // namespace

array gsplat_sh_camera_colors_forward(int degree, const array& means_in, const array& viewmats_in, const array& dc_in,
                                      const array& rest_in, const array& radii_in, StreamOrDevice s) {
  const CamDims d = validate_camera("sh_camera_colors_forward", degree, means_in, viewmats_in, dc_in, rest_in);
  const c10::DeviceGuard guard(means_in.device());
  const array means = contig(means_in), viewmats = contig(viewmats_in), dc = contig(dc_in), rest = contig(rest_in);
  array radii;
  const int32_t* rp = camera_radii(radii_in, d, means, radii, "sh_camera_colors_forward");
  std::vector<int64_t> shape(means.sizes().begin(), means.sizes().end() - 2);
  shape.insert(shape.end(), {d.C, d.N, 3});
  array colors = at::empty(shape, f32_like(means));
  check(gsplat_hip_sh_camera_colors_fwd(degree, means.data_ptr<float>(), viewmats.data_ptr<float>(),
                                        dc.data_ptr<float>(), d.R > 0 ? rest.data_ptr<float>() : nullptr, rp, d.B,
                                        d.C, d.N, d.R, colors.data_ptr<float>(), stream_for(s, means)));
  return colors;
}

std::vector<array> gsplat_sh_camera_colors_backward(int degree, const array& means_in, const array& viewmats_in,
                                                    const array& dc_in, const array& rest_in,
                                                    const array& v_colors_in, StreamOrDevice s) {
  const CamDims d = validate_camera("sh_camera_colors_backward", degree, means_in, viewmats_in, dc_in, rest_in);
  if (v_colors_in.numel() != d.B * d.C * d.N * 3 || v_colors_in.scalar_type() != at::kFloat)
    throw std::runtime_error("v_colors must have shape [..., C, N, 3] (float32).");
  require_device(v_colors_in, "v_colors");
  const c10::DeviceGuard guard(means_in.device());
  const array means = contig(means_in), viewmats = contig(viewmats_in), dc = contig(dc_in), rest = contig(rest_in);
  const array v_colors = contig(v_colors_in);
  array v_means = at::empty(means.sizes(), f32_like(means));
  array v_dc = at::empty(dc.sizes(), f32_like(means));
  array v_rest = at::empty(rest.sizes(), f32_like(means));
  check(gsplat_hip_sh_camera_colors_bwd(degree, means.data_ptr<float>(), viewmats.data_ptr<float>(),
                                        dc.data_ptr<float>(), d.R > 0 ? rest.data_ptr<float>() : nullptr,
                                        v_colors.data_ptr<float>(), d.B, d.C, d.N, d.R, v_means.data_ptr<float>(),
                                        v_dc.data_ptr<float>(), d.R > 0 ? v_rest.data_ptr<float>() : nullptr,
                                        stream_for(s, means)));
  return {v_means, v_dc, v_rest};
}

namespace {

// The packed count workspace (uint8, the packed projection's "rank" output)
// and the packed row count of the packed camera colour functions.
void check_packed_rank(const array& rank, int64_t nnz, const CamDims& d, const array& means, const char* what) {
  const std::string o(what);
  if (rank.scalar_type() != at::kByte || rank.dim() != 1)
    throw std::runtime_error(o + ": rank must be the packed projection's uint8 workspace.");
  if (rank.device() != means.device()) throw std::runtime_error(o + ": rank must be on the means' device.");
  if (nnz < 0 || nnz > d.B * d.C * d.N) throw std::runtime_error(o + ": invalid packed row count.");
}

}  // namespace

array gsplat_sh_camera_colors_packed_forward(int degree, const array& means_in, const array& viewmats_in,
                                             const array& dc_in, const array& rest_in, const array& rank_in,
                                             int64_t nnz, StreamOrDevice s) {
  const char* what = "sh_camera_colors_packed_forward";
  const CamDims d = validate_camera(what, degree, means_in, viewmats_in, dc_in, rest_in);
  check_packed_rank(rank_in, nnz, d, means_in, what);
  const c10::DeviceGuard guard(means_in.device());
  const array means = contig(means_in), viewmats = contig(viewmats_in), dc = contig(dc_in), rest = contig(rest_in);
  const array rank = contig(rank_in);
  array rows = at::empty({nnz, 3}, f32_like(means));
  check(gsplat_hip_sh_camera_colors_packed_fwd(
      degree, means.data_ptr<float>(), viewmats.data_ptr<float>(), dc.data_ptr<float>(),
      d.R > 0 ? rest.data_ptr<float>() : nullptr, rank.numel() ? rank.data_ptr<uint8_t>() : nullptr,
      static_cast<size_t>(rank.numel()), nnz, d.B, d.C, d.N, d.R, rows.data_ptr<float>(), stream_for(s, means)));
  return rows;
}

std::vector<array> gsplat_sh_camera_colors_packed_backward(int degree, const array& means_in,
                                                           const array& viewmats_in, const array& dc_in,
                                                           const array& rest_in, const array& rank_in,
                                                           const array& v_rows_in, StreamOrDevice s) {
  const char* what = "sh_camera_colors_packed_backward";
  const CamDims d = validate_camera(what, degree, means_in, viewmats_in, dc_in, rest_in);
  const int64_t nnz = v_rows_in.dim() == 2 ? v_rows_in.size(0) : -1;
  if (nnz < 0 || v_rows_in.size(1) != 3 || v_rows_in.scalar_type() != at::kFloat)
    throw std::runtime_error(std::string(what) + ": v_colors must have shape [nnz, 3] (float32).");
  require_device(v_rows_in, "v_colors");
  check_packed_rank(rank_in, nnz, d, means_in, what);
  const c10::DeviceGuard guard(means_in.device());
  const array means = contig(means_in), viewmats = contig(viewmats_in), dc = contig(dc_in), rest = contig(rest_in);
  const array rank = contig(rank_in), v_rows = contig(v_rows_in);
  array v_means = at::empty(means.sizes(), f32_like(means));
  array v_dc = at::empty(dc.sizes(), f32_like(means));
  array v_rest = at::empty(rest.sizes(), f32_like(means));
  check(gsplat_hip_sh_camera_colors_packed_bwd(
      degree, means.data_ptr<float>(), viewmats.data_ptr<float>(), dc.data_ptr<float>(),
      d.R > 0 ? rest.data_ptr<float>() : nullptr, rank.numel() ? rank.data_ptr<uint8_t>() : nullptr,
      static_cast<size_t>(rank.numel()), nnz ? v_rows.data_ptr<float>() : nullptr, nnz, d.B, d.C, d.N, d.R,
      v_means.data_ptr<float>(), v_dc.data_ptr<float>(), d.R > 0 ? v_rest.data_ptr<float>() : nullptr,
      stream_for(s, means)));
  return {v_means, v_dc, v_rest};
}

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
