// Python module `_gsplat_core`: the reference binding's surface
// (gsplat_core/binding/binding.cpp:447-534) -- same function names, dict
// inputs, keyword defaults, output dict keys and "missing optional key ->
// empty array" convention -- over torch tensors on a ROCm device. Built
// with pybind11 (nanobind is not available in this toolchain).
#include <torch/extension.h>

#include <stdexcept>
#include <string>
#include <unordered_map>

#include "gsplat_core.h"

namespace py = pybind11;
using TensorMap = std::unordered_map<std::string, at::Tensor>;

namespace {

// binding.cpp:26-35
const at::Tensor& require_key(const TensorMap& inputs, const char* key) {
  auto it = inputs.find(key);
  if (it == inputs.end()) throw std::runtime_error(std::string("gsplat_core binding missing input: ") + key);
  return it->second;
}

// absent optional input -> undefined tensor
at::Tensor get_or_undefined(const TensorMap& inputs, const char* key) {
  auto it = inputs.find(key);
  return it == inputs.end() ? at::Tensor() : it->second;
}

// binding.cpp:37-45: absent optional input -> empty float32 array
at::Tensor get_or_empty(const TensorMap& inputs, const char* key) {
  auto it = inputs.find(key);
  if (it == inputs.end()) return at::empty({0}, at::TensorOptions().dtype(at::kFloat));
  return it->second;
}

py::dict projection_ewa_3dgs_fused_forward(const TensorMap& inputs, int image_width, int image_height, float eps2d,
                                           float near_plane, float far_plane, float radius_clip,
                                           bool calc_compensations, int camera_model) {
  gsplat_core::ProjectionEWA3DGSFusedInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.covars = get_or_empty(inputs, "covars");
  in.quats = get_or_empty(inputs, "quats");
  in.scales = get_or_empty(inputs, "scales");
  in.opacities = get_or_empty(inputs, "opacities");
  in.viewspace_points = get_or_empty(inputs, "viewspace_points");
  in.params = {image_width, image_height, eps2d, near_plane, far_plane, radius_clip, calc_compensations,
               camera_model, in.covars.numel() != 0, in.opacities.numel() != 0};
  auto out = gsplat_core::gsplat_projection_ewa_3dgs_fused(in);
  py::dict r;
  r["radii"] = out[gsplat_core::kRadii];
  r["means2d"] = out[gsplat_core::kMeans2D];
  r["depths"] = out[gsplat_core::kDepths];
  r["conics"] = out[gsplat_core::kConics];
  r["compensations"] = out[gsplat_core::kCompensations];
  r["viewspace_points"] = in.viewspace_points;
  return r;
}

// binding.cpp:119-186. The reference evaluates this entry point on the CPU;
// here it runs the GPU kernel with the same fixed parameters.
py::dict projection_ewa_3dgs_fused_backward(const TensorMap& inputs, const TensorMap& forward_outputs,
                                            const TensorMap& cotangents, int image_width, int image_height,
                                            float eps2d, int camera_model, bool viewmats_requires_grad) {
  gsplat_core::ProjectionEWA3DGSFusedBackwardInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.covars = get_or_empty(inputs, "covars");
  in.quats = get_or_empty(inputs, "quats");
  in.scales = get_or_empty(inputs, "scales");
  in.radii = require_key(forward_outputs, "radii");
  in.conics = require_key(forward_outputs, "conics");
  in.compensations = get_or_empty(forward_outputs, "compensations");
  in.v_means2d = require_key(cotangents, "v_means2d");
  in.v_depths = get_or_empty(cotangents, "v_depths");  // absent = zeros
  in.v_conics = require_key(cotangents, "v_conics");
  in.v_compensations = get_or_empty(cotangents, "v_compensations");
  const bool use_covars = in.covars.numel() != 0;
  in.params = {image_width, image_height, eps2d, -1.0e20f, 1.0e20f, 0.0f, in.compensations.numel() != 0,
               camera_model, use_covars, false};
  in.viewmats_requires_grad = viewmats_requires_grad;
  auto out = gsplat_core::gsplat_projection_ewa_3dgs_fused_backward(in);
  py::dict r;
  r["v_means"] = out[gsplat_core::kProjectionVMeans];
  if (use_covars) {
    r["v_covars"] = out[gsplat_core::kProjectionVCovars];
  } else {
    r["v_quats"] = out[gsplat_core::kProjectionVQuats];
    r["v_scales"] = out[gsplat_core::kProjectionVScales];
  }
  if (viewmats_requires_grad) r["v_viewmats"] = out[gsplat_core::kProjectionVViewmats];
  return r;
}

// Packed layout (the reference's intended projection_ewa_3dgs_packed_forward,
// note/gsplat_cuda_source_map.md:273-315; upstream gsplat's
// fully_fused_projection(packed=True)).
py::dict projection_ewa_3dgs_packed_forward(const TensorMap& inputs, int image_width, int image_height, float eps2d,
                                            float near_plane, float far_plane, float radius_clip,
                                            bool calc_compensations, int camera_model) {
  gsplat_core::ProjectionEWA3DGSFusedInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.covars = get_or_empty(inputs, "covars");
  in.quats = get_or_empty(inputs, "quats");
  in.scales = get_or_empty(inputs, "scales");
  in.opacities = get_or_empty(inputs, "opacities");
  in.params = {image_width, image_height, eps2d, near_plane, far_plane, radius_clip, calc_compensations,
               camera_model, in.covars.numel() != 0, in.opacities.numel() != 0};
  auto out = gsplat_core::gsplat_projection_ewa_3dgs_packed(in);
  py::dict r;
  r["batch_ids"] = out[gsplat_core::kPackedBatchIds];
  r["camera_ids"] = out[gsplat_core::kPackedCameraIds];
  r["gaussian_ids"] = out[gsplat_core::kPackedGaussianIds];
  r["indptr"] = out[gsplat_core::kPackedIndptr];
  r["radii"] = out[gsplat_core::kPackedRadii];
  r["means2d"] = out[gsplat_core::kPackedMeans2D];
  r["depths"] = out[gsplat_core::kPackedDepths];
  r["conics"] = out[gsplat_core::kPackedConics];
  r["compensations"] = out[gsplat_core::kPackedCompensations];
  return r;
}

py::dict projection_ewa_3dgs_packed_backward(const TensorMap& inputs, const TensorMap& forward_outputs,
                                             const TensorMap& cotangents, int image_width, int image_height,
                                             float eps2d, int camera_model, bool viewmats_requires_grad) {
  gsplat_core::ProjectionEWA3DGSPackedBackwardInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.covars = get_or_empty(inputs, "covars");
  in.quats = get_or_empty(inputs, "quats");
  in.scales = get_or_empty(inputs, "scales");
  in.batch_ids = get_or_empty(forward_outputs, "batch_ids");
  in.camera_ids = require_key(forward_outputs, "camera_ids");
  in.gaussian_ids = require_key(forward_outputs, "gaussian_ids");
  in.conics = require_key(forward_outputs, "conics");
  in.compensations = get_or_empty(forward_outputs, "compensations");
  in.v_means2d = require_key(cotangents, "v_means2d");
  in.v_depths = get_or_empty(cotangents, "v_depths");  // absent = zeros
  in.v_conics = require_key(cotangents, "v_conics");
  in.v_compensations = get_or_empty(cotangents, "v_compensations");
  const bool use_covars = in.covars.numel() != 0;
  in.params = {image_width, image_height, eps2d, -1.0e20f, 1.0e20f, 0.0f, in.compensations.numel() != 0,
               camera_model, use_covars, false};
  in.viewmats_requires_grad = viewmats_requires_grad;
  auto out = gsplat_core::gsplat_projection_ewa_3dgs_packed_backward(in);
  py::dict r;
  r["v_means"] = out[gsplat_core::kProjectionVMeans];
  if (use_covars) {
    r["v_covars"] = out[gsplat_core::kProjectionVCovars];
  } else {
    r["v_quats"] = out[gsplat_core::kProjectionVQuats];
    r["v_scales"] = out[gsplat_core::kProjectionVScales];
  }
  if (viewmats_requires_grad) r["v_viewmats"] = out[gsplat_core::kProjectionVViewmats];
  return r;
}

gsplat_core::IntersectTileInput intersect_input(const TensorMap& inputs, int I, int tile_size, int tile_width,
                                                int tile_height, bool sort, bool segmented) {
  gsplat_core::IntersectTileInput in;
  in.means2d = require_key(inputs, "means2d");
  in.radii = require_key(inputs, "radii");
  in.depths = require_key(inputs, "depths");
  in.conics = get_or_empty(inputs, "conics");
  in.opacities = get_or_empty(inputs, "opacities");
  in.image_ids = get_or_empty(inputs, "image_ids");
  in.gaussian_ids = get_or_empty(inputs, "gaussian_ids");
  in.params = {I,
               tile_size,
               tile_width,
               tile_height,
               sort,
               segmented,
               in.image_ids.numel() != 0 || in.gaussian_ids.numel() != 0,
               in.conics.numel() != 0,
               in.opacities.numel() != 0};
  return in;
}

py::dict intersect_tile_forward(const TensorMap& inputs, int I, int tile_size, int tile_width, int tile_height,
                                bool sort, bool segmented) {
  auto out = gsplat_core::gsplat_intersect_tile(
      intersect_input(inputs, I, tile_size, tile_width, tile_height, sort, segmented));
  py::dict r;
  r["tiles_per_gauss"] = out[gsplat_core::kTilesPerGauss];
  r["isect_ids"] = out[gsplat_core::kIsectIds];
  r["flatten_ids"] = out[gsplat_core::kFlattenIds];
  return r;
}

// intersect_tile_forward (sorted) + intersect_offset_forward in one call: the
// dict also holds "tile_offsets" [I, tile_height, tile_width].
py::dict intersect_tile_offsets_forward(const TensorMap& inputs, int I, int tile_size, int tile_width,
                                        int tile_height) {
  auto out = gsplat_core::gsplat_intersect_tile_with_offsets(
      intersect_input(inputs, I, tile_size, tile_width, tile_height, true, false));
  py::dict r;
  r["tiles_per_gauss"] = out[gsplat_core::kTilesPerGauss];
  r["isect_ids"] = out[gsplat_core::kIsectIds];
  r["flatten_ids"] = out[gsplat_core::kFlattenIds];
  r["tile_offsets"] = out[3];
  return r;
}

// The same in two calls around the count read-back (gsplat_intersect_tile_
// offsets_begin / _end): work queued on the stream between them runs while
// the host waits for the count.
struct PendingIntersectHandle {
  std::shared_ptr<gsplat_core::PendingIntersect> p;
};

PendingIntersectHandle intersect_tile_offsets_begin(const TensorMap& inputs, int I, int tile_size, int tile_width,
                                                    int tile_height) {
  return {gsplat_core::gsplat_intersect_tile_offsets_begin(
      intersect_input(inputs, I, tile_size, tile_width, tile_height, true, false))};
}

py::dict intersect_tile_offsets_end(const PendingIntersectHandle& h) {
  auto out = gsplat_core::gsplat_intersect_tile_offsets_end(h.p);
  py::dict r;
  r["tiles_per_gauss"] = out[gsplat_core::kTilesPerGauss];
  r["isect_ids"] = out[gsplat_core::kIsectIds];
  r["flatten_ids"] = out[gsplat_core::kFlattenIds];
  r["tile_offsets"] = out[3];
  return r;
}

at::Tensor intersect_offset_forward(const at::Tensor& isect_ids, int I, int tile_width, int tile_height) {
  return gsplat_core::gsplat_intersect_offset(isect_ids, I, tile_width, tile_height);
}

// upstream gsplat's rasterize_to_indices_in_range (the reference's planned
// rasterize_to_indices_3dgs_forward, note/gsplat_cuda_source_map.md:494-545)
py::dict rasterize_to_indices_3dgs_forward(const TensorMap& inputs, int64_t range_start, int64_t range_end,
                                           int image_width, int image_height, int tile_size) {
  auto out = gsplat_core::gsplat_rasterize_to_indices_3dgs(
      range_start, range_end, get_or_empty(inputs, "transmittances"), require_key(inputs, "means2d"),
      require_key(inputs, "conics"), require_key(inputs, "opacities"), image_width, image_height, tile_size,
      require_key(inputs, "tile_offsets"), require_key(inputs, "flatten_ids"));
  py::dict r;
  r["gaussian_ids"] = out[0];
  r["indices"] = out[1];
  return r;
}

py::dict rasterize_to_pixels_3dgs_forward(const TensorMap& inputs, int image_width, int image_height, int tile_size) {
  gsplat_core::RasterizeToPixels3DGSInput in;
  in.means2d = require_key(inputs, "means2d");
  in.conics = require_key(inputs, "conics");
  in.colors = require_key(inputs, "colors");
  in.opacities = require_key(inputs, "opacities");
  in.tile_offsets = require_key(inputs, "tile_offsets");
  in.flatten_ids = require_key(inputs, "flatten_ids");
  in.backgrounds = get_or_empty(inputs, "backgrounds");
  in.masks = get_or_empty(inputs, "masks");
  in.params = {image_width, image_height, tile_size, in.backgrounds.numel() != 0, in.masks.numel() != 0,
               in.means2d.dim() == 2};
  auto out = gsplat_core::gsplat_rasterize_to_pixels_3dgs(in);
  py::dict r;
  r["render_colors"] = out[gsplat_core::kRenderColors];
  r["render_alphas"] = out[gsplat_core::kRenderAlphas];
  r["last_ids"] = out[gsplat_core::kLastIds];
  return r;
}

py::dict rasterize_to_pixels_3dgs_backward(const TensorMap& inputs, const TensorMap& forward_outputs,
                                           const TensorMap& cotangents, int image_width, int image_height,
                                           int tile_size, bool absgrad) {
  gsplat_core::RasterizeToPixels3DGSBackwardInput in;
  in.means2d = require_key(inputs, "means2d");
  in.conics = require_key(inputs, "conics");
  in.colors = require_key(inputs, "colors");
  in.opacities = require_key(inputs, "opacities");
  in.tile_offsets = require_key(inputs, "tile_offsets");
  in.flatten_ids = require_key(inputs, "flatten_ids");
  in.render_alphas = require_key(forward_outputs, "render_alphas");
  in.last_ids = require_key(forward_outputs, "last_ids");
  in.v_render_colors = require_key(cotangents, "v_render_colors");
  in.v_render_alphas = get_or_empty(cotangents, "v_render_alphas");  // absent = zeros
  in.backgrounds = get_or_empty(inputs, "backgrounds");
  in.masks = get_or_empty(inputs, "masks");
  in.params = {image_width, image_height, tile_size, in.backgrounds.numel() != 0, in.masks.numel() != 0,
               in.means2d.dim() == 2};
  in.absgrad = absgrad;
  auto out = gsplat_core::gsplat_rasterize_to_pixels_3dgs_backward(in);
  py::dict r;
  if (absgrad) r["v_means2d_abs"] = out[gsplat_core::kRasterVMeans2DAbs];
  r["v_means2d"] = out[gsplat_core::kRasterVMeans2D];
  r["v_conics"] = out[gsplat_core::kRasterVConics];
  r["v_colors"] = out[gsplat_core::kRasterVColors];
  r["v_opacities"] = out[gsplat_core::kRasterVOpacities];
  if (in.backgrounds.numel() != 0) r["v_backgrounds"] = out[gsplat_core::kRasterVBackgrounds];
  return r;
}

at::Tensor spherical_harmonics_forward(int degrees_to_use, const TensorMap& inputs) {
  gsplat_core::SphericalHarmonicsInput in;
  in.degrees_to_use = degrees_to_use;
  in.dirs = require_key(inputs, "dirs");
  in.coeffs = require_key(inputs, "coeffs");
  in.masks = get_or_empty(inputs, "masks");
  in.use_masks = in.masks.numel() != 0;
  return gsplat_core::gsplat_spherical_harmonics_forward(in);
}

py::dict spherical_harmonics_backward(int degrees_to_use, const TensorMap& inputs, const TensorMap& cotangents,
                                      bool compute_v_dirs) {
  gsplat_core::SphericalHarmonicsBackwardInput in;
  in.degrees_to_use = degrees_to_use;
  in.dirs = require_key(inputs, "dirs");
  in.coeffs = require_key(inputs, "coeffs");
  in.v_colors = require_key(cotangents, "v_colors");
  in.masks = get_or_empty(inputs, "masks");
  in.use_masks = in.masks.numel() != 0;
  in.compute_v_dirs = compute_v_dirs;
  auto out = gsplat_core::gsplat_spherical_harmonics_backward(in);
  py::dict r;
  if (compute_v_dirs) r["v_dirs"] = out[gsplat_core::kSHVDirs];
  r["v_coeffs"] = out[gsplat_core::kSHVCoeffs];
  return r;
}

py::dict quat_scale_to_covar_preci_forward(const TensorMap& inputs, bool compute_covar, bool compute_preci,
                                           bool triu) {
  gsplat_core::QuatScaleToCovarPreciInput in;
  in.quats = require_key(inputs, "quats");
  in.scales = require_key(inputs, "scales");
  in.compute_covar = compute_covar;
  in.compute_preci = compute_preci;
  in.triu = triu;
  auto out = gsplat_core::gsplat_quat_scale_to_covar_preci_forward(in);
  py::dict r;
  r["covars"] = out[gsplat_core::kCovars];
  r["precis"] = out[gsplat_core::kPrecis];
  return r;
}

py::dict quat_scale_to_covar_preci_backward(const TensorMap& inputs, const TensorMap& cotangents, bool triu) {
  gsplat_core::QuatScaleToCovarPreciBackwardInput in;
  in.quats = require_key(inputs, "quats");
  in.scales = require_key(inputs, "scales");
  in.v_covars = get_or_empty(cotangents, "v_covars");
  in.v_precis = get_or_empty(cotangents, "v_precis");
  in.triu = triu;
  in.use_v_covars = in.v_covars.numel() != 0;
  in.use_v_precis = in.v_precis.numel() != 0;
  auto out = gsplat_core::gsplat_quat_scale_to_covar_preci_backward(in);
  py::dict r;
  r["v_quats"] = out[gsplat_core::kVQuats];
  r["v_scales"] = out[gsplat_core::kVScales];
  return r;
}

// Caller-side SH glue fused into the kernels (addition to the reference
// surface; see gsplat_sh_camera_colors_forward).
// Optional forward input "radii" (the projection's): rows no camera sees
// are skipped (colour 0).
at::Tensor sh_camera_colors_forward(int degrees_to_use, const TensorMap& inputs) {
  return gsplat_core::gsplat_sh_camera_colors_forward(
      degrees_to_use, require_key(inputs, "means"), require_key(inputs, "viewmats"), require_key(inputs, "features_dc"),
      require_key(inputs, "features_rest"), get_or_undefined(inputs, "radii"));
}

py::dict sh_camera_colors_backward(int degrees_to_use, const TensorMap& inputs, const TensorMap& cotangents) {
  auto out = gsplat_core::gsplat_sh_camera_colors_backward(
      degrees_to_use, require_key(inputs, "means"), require_key(inputs, "viewmats"), require_key(inputs, "features_dc"),
      require_key(inputs, "features_rest"), require_key(cotangents, "v_colors"));
  py::dict r;
  r["v_means"] = out[0];
  r["v_features_dc"] = out[1];
  r["v_features_rest"] = out[2];
  return r;
}

// The packed layout's camera colours: inputs as above plus "rank" (the
// packed projection's count workspace); the forward returns [nnz, 3] rows.
at::Tensor sh_camera_colors_packed_forward(int degrees_to_use, const TensorMap& inputs, int64_t nnz) {
  return gsplat_core::gsplat_sh_camera_colors_packed_forward(
      degrees_to_use, require_key(inputs, "means"), require_key(inputs, "viewmats"), require_key(inputs, "features_dc"),
      require_key(inputs, "features_rest"), require_key(inputs, "rank"), nnz);
}

py::dict sh_camera_colors_packed_backward(int degrees_to_use, const TensorMap& inputs, const TensorMap& cotangents) {
  auto out = gsplat_core::gsplat_sh_camera_colors_packed_backward(
      degrees_to_use, require_key(inputs, "means"), require_key(inputs, "viewmats"), require_key(inputs, "features_dc"),
      require_key(inputs, "features_rest"), require_key(inputs, "rank"), require_key(cotangents, "v_colors"));
  py::dict r;
  r["v_means"] = out[0];
  r["v_features_dc"] = out[1];
  r["v_features_rest"] = out[2];
  return r;
}

// Training-step glue fused into kernels (additions to the reference surface;
// see gsplat_training_glue.h).
py::dict gaussian_activations_forward(const TensorMap& inputs) {
  auto out = gsplat_core::gsplat_gaussian_activations_forward(
      get_or_empty(inputs, "quats"), get_or_empty(inputs, "log_scales"), get_or_empty(inputs, "opacity_logits"));
  py::dict r;
  r["quats"] = out[0];
  r["scales"] = out[1];
  r["opacities"] = out[2];
  return r;
}

// Activated projection: the activations fused into the projection. inputs:
// means, quats (raw), log_scales, opacity_logits (optional), viewmats, Ks.
py::dict activated_projection_forward(const TensorMap& inputs, int image_width, int image_height, float eps2d,
                                      float near_plane, float far_plane, float radius_clip, bool calc_compensations,
                                      int camera_model, bool opacities_in_projection) {
  gsplat_core::ProjectionEWA3DGSFusedInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.quats = require_key(inputs, "quats");
  in.scales = require_key(inputs, "log_scales");
  in.opacities = get_or_empty(inputs, "opacity_logits");
  in.params = {image_width, image_height, eps2d, near_plane, far_plane, radius_clip, calc_compensations,
               camera_model, false, opacities_in_projection && in.opacities.numel() != 0};
  auto out = gsplat_core::gsplat_activated_projection_forward(in);
  py::dict r;
  r["radii"] = out[gsplat_core::kRadii];
  r["means2d"] = out[gsplat_core::kMeans2D];
  r["depths"] = out[gsplat_core::kDepths];
  r["conics"] = out[gsplat_core::kConics];
  r["compensations"] = out[gsplat_core::kCompensations];
  r["opacities"] = out[5];
  return r;
}

// Activated packed projection: inputs as activated_projection_forward; the
// packed rows plus per-row "opacities" and the "rank" the backward reads.
py::dict activated_projection_packed_forward(const TensorMap& inputs, int image_width, int image_height,
                                             float eps2d, float near_plane, float far_plane, float radius_clip,
                                             bool calc_compensations, int camera_model,
                                             bool opacities_in_projection) {
  gsplat_core::ProjectionEWA3DGSFusedInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.quats = require_key(inputs, "quats");
  in.scales = require_key(inputs, "log_scales");
  in.opacities = get_or_empty(inputs, "opacity_logits");
  in.params = {image_width, image_height, eps2d, near_plane, far_plane, radius_clip, calc_compensations,
               camera_model, false, opacities_in_projection && in.opacities.numel() != 0};
  auto out = gsplat_core::gsplat_activated_projection_packed_forward(in);
  py::dict r;
  const char* keys[] = {"batch_ids", "camera_ids", "gaussian_ids", "indptr", "radii", "means2d",
                        "depths",    "conics",     "compensations", "opacities", "rank"};
  for (size_t i = 0; i < out.size(); ++i) r[keys[i]] = out[i];
  return r;
}

// forward_outputs: conics, rank (compensations optional); cotangents per row
// (v_depths, v_compensations, v_opacities optional).
py::dict activated_projection_packed_backward(const TensorMap& inputs, const TensorMap& forward_outputs,
                                              const TensorMap& cotangents, int image_width, int image_height,
                                              float eps2d, int camera_model, bool viewmats_requires_grad,
                                              bool viewspace_requires_grad) {
  gsplat_core::ProjectionEWA3DGSPackedBackwardInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.quats = require_key(inputs, "quats");
  in.scales = require_key(inputs, "log_scales");
  in.conics = require_key(forward_outputs, "conics");
  in.compensations = get_or_empty(forward_outputs, "compensations");
  in.v_means2d = require_key(cotangents, "v_means2d");
  in.v_depths = get_or_empty(cotangents, "v_depths");
  in.v_conics = require_key(cotangents, "v_conics");
  in.v_compensations = get_or_empty(cotangents, "v_compensations");
  in.params = {image_width, image_height, eps2d, -1.0e20f, 1.0e20f, 0.0f, in.compensations.numel() != 0,
               camera_model, false, false};
  in.viewmats_requires_grad = viewmats_requires_grad;
  auto out = gsplat_core::gsplat_activated_projection_packed_backward(
      in, require_key(forward_outputs, "rank"), get_or_empty(inputs, "opacity_logits"),
      get_or_empty(cotangents, "v_opacities"), viewspace_requires_grad);
  py::dict r;
  r["v_means"] = out[0];
  r["v_quats"] = out[1];
  r["v_log_scales"] = out[2];
  r["v_opacity_logits"] = out[3];
  if (viewmats_requires_grad) r["v_viewmats"] = out[4];
  if (viewspace_requires_grad) r["v_viewspace"] = out[5];
  return r;
}

// Packed rows of dense [B, C, N, K] values (batch_ids optional with B = 1).
at::Tensor packed_rows_gather(const at::Tensor& dense, const TensorMap& ids) {
  return gsplat_core::gsplat_packed_rows_gather(dense, get_or_empty(ids, "batch_ids"), require_key(ids, "camera_ids"),
                                                require_key(ids, "gaussian_ids"));
}

// The adjoint: rows at their slots of a dense [B, C, N, K] array, zeros
// elsewhere (rank: the activated packed forward's).
at::Tensor packed_rows_scatter(const at::Tensor& rows, const at::Tensor& rank, int64_t B, int64_t C, int64_t N) {
  return gsplat_core::gsplat_packed_rows_scatter(rows, rank, B, C, N);
}

py::dict activated_projection_backward(const TensorMap& inputs, const TensorMap& forward_outputs,
                                       const TensorMap& cotangents, int image_width, int image_height, float eps2d,
                                       int camera_model, bool viewmats_requires_grad) {
  gsplat_core::ProjectionEWA3DGSFusedBackwardInput in;
  in.means = require_key(inputs, "means");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.quats = require_key(inputs, "quats");
  in.scales = require_key(inputs, "log_scales");
  in.radii = require_key(forward_outputs, "radii");
  in.conics = require_key(forward_outputs, "conics");
  in.compensations = get_or_empty(forward_outputs, "compensations");
  in.v_means2d = require_key(cotangents, "v_means2d");
  in.v_depths = get_or_empty(cotangents, "v_depths");  // absent = zeros
  in.v_conics = require_key(cotangents, "v_conics");
  in.v_compensations = get_or_empty(cotangents, "v_compensations");
  in.params = {image_width, image_height, eps2d, -1.0e20f, 1.0e20f, 0.0f, in.compensations.numel() != 0,
               camera_model, false, false};
  in.viewmats_requires_grad = viewmats_requires_grad;
  auto out = gsplat_core::gsplat_activated_projection_backward(in, get_or_empty(inputs, "opacity_logits"),
                                                               get_or_empty(cotangents, "v_opacities"));
  py::dict r;
  r["v_means"] = out[0];
  r["v_quats"] = out[1];
  r["v_log_scales"] = out[2];
  r["v_opacity_logits"] = out[3];
  if (viewmats_requires_grad) r["v_viewmats"] = out[4];
  return r;
}

py::dict gaussian_activations_backward(const TensorMap& inputs, const TensorMap& forward_outputs,
                                       const TensorMap& cotangents) {
  auto out = gsplat_core::gsplat_gaussian_activations_backward(
      get_or_empty(inputs, "quats"), get_or_empty(forward_outputs, "scales"),
      get_or_empty(forward_outputs, "opacities"), get_or_empty(cotangents, "v_quats"),
      get_or_empty(cotangents, "v_scales"), get_or_empty(cotangents, "v_opacities"));
  py::dict r;
  r["v_quats"] = out[0];
  r["v_log_scales"] = out[1];
  r["v_opacity_logits"] = out[2];
  return r;
}

at::Tensor l1_loss_forward(const at::Tensor& image, const at::Tensor& target) {
  return gsplat_core::gsplat_l1_loss_forward(image, target);
}

py::tuple l1_loss_backward(const at::Tensor& image, const at::Tensor& target, const at::Tensor& grad) {
  auto out = gsplat_core::gsplat_l1_loss_backward(image, target, grad);
  return py::make_tuple(out[0], out[1]);
}

py::tuple image_loss_forward(const at::Tensor& image, const at::Tensor& target, int window_size, bool with_maps) {
  auto out = gsplat_core::gsplat_image_loss_forward(image, target, window_size, with_maps);
  return py::make_tuple(out[0], out[1]);
}

at::Tensor image_loss_backward(const at::Tensor& image, const at::Tensor& target, const at::Tensor& maps,
                               int window_size, const at::Tensor& g_l1, const at::Tensor& g_ssim) {
  return gsplat_core::gsplat_image_loss_backward(image, target, maps, window_size, g_l1, g_ssim);
}

// The RGB render step in one call per direction (gsplat_render.h; no
// counterpart in the reference binding): inputs means, quats, log_scales,
// opacity_logits, colors, viewmats, Ks and optional backgrounds; the forward
// returns the images, the intersections and what the backward reads back.
gsplat_core::RenderRGBInput render_rgb_input(const TensorMap& inputs, int image_width, int image_height,
                                             int tile_size, float eps2d, float near_plane, float far_plane,
                                             bool opacities_in_projection, bool accutile) {
  gsplat_core::RenderRGBInput in;
  in.means = require_key(inputs, "means");
  in.quats = require_key(inputs, "quats");
  in.log_scales = require_key(inputs, "log_scales");
  in.opacity_logits = require_key(inputs, "opacity_logits");
  in.colors = require_key(inputs, "colors");
  in.viewmats = require_key(inputs, "viewmats");
  in.Ks = require_key(inputs, "Ks");
  in.backgrounds = get_or_empty(inputs, "backgrounds");
  in.image_width = image_width;
  in.image_height = image_height;
  in.tile_size = tile_size;
  in.eps2d = eps2d;
  in.near_plane = near_plane;
  in.far_plane = far_plane;
  in.opacities_in_projection = opacities_in_projection;
  in.accutile = accutile;
  return in;
}

const char* const kRenderRGBKeys[] = {"render_colors", "render_alphas", "last_ids", "radii", "means2d", "conics",
                                      "opacities", "tiles_per_gauss", "isect_ids", "flatten_ids", "tile_offsets"};

py::dict render_rgb_forward(const TensorMap& inputs, int image_width, int image_height, int tile_size, float eps2d,
                            float near_plane, float far_plane, bool opacities_in_projection, bool accutile) {
  auto out = gsplat_core::gsplat_render_rgb_forward(render_rgb_input(
      inputs, image_width, image_height, tile_size, eps2d, near_plane, far_plane, opacities_in_projection, accutile));
  py::dict r;
  for (size_t i = 0; i < out.size(); ++i) r[kRenderRGBKeys[i]] = out[i];
  return r;
}

py::dict render_rgb_backward(const TensorMap& inputs, const TensorMap& forward_outputs, const TensorMap& cotangents,
                             int image_width, int image_height, int tile_size, float eps2d, bool accutile,
                             bool viewmats_requires_grad) {
  const auto in = render_rgb_input(inputs, image_width, image_height, tile_size, eps2d, 0.01f, 1e10f, false, accutile);
  std::vector<at::Tensor> fwd;
  for (const char* k : kRenderRGBKeys) fwd.push_back(require_key(forward_outputs, k));
  auto out = gsplat_core::gsplat_render_rgb_backward(in, fwd, require_key(cotangents, "v_render_colors"),
                                                     get_or_empty(cotangents, "v_render_alphas"),
                                                     viewmats_requires_grad);
  py::dict r;
  r["v_means"] = out[0];
  r["v_quats"] = out[1];
  r["v_log_scales"] = out[2];
  r["v_opacity_logits"] = out[3];
  r["v_colors"] = out[4];
  if (viewmats_requires_grad) r["v_viewmats"] = out[5];
  return r;
}

// Loss and gradients of the RGB step with the L1 image loss in one call
// (gsplat_render_rgb_l1_value_and_grad): {"loss", the forward's keys,
// "v_means", "v_quats", "v_log_scales", "v_opacity_logits", "v_colors"}.
py::dict render_rgb_l1_value_and_grad(const TensorMap& inputs, const at::Tensor& target, int image_width,
                                      int image_height, int tile_size, float eps2d, float near_plane, float far_plane,
                                      bool opacities_in_projection, bool accutile) {
  auto out = gsplat_core::gsplat_render_rgb_l1_value_and_grad(
      render_rgb_input(inputs, image_width, image_height, tile_size, eps2d, near_plane, far_plane,
                       opacities_in_projection, accutile),
      target);
  py::dict r;
  r["loss"] = out[0];
  const size_t nf = sizeof(kRenderRGBKeys) / sizeof(kRenderRGBKeys[0]);
  for (size_t i = 0; i < nf; ++i) r[kRenderRGBKeys[i]] = out[1 + i];
  const char* const grads[] = {"v_means", "v_quats", "v_log_scales", "v_opacity_logits", "v_colors"};
  for (size_t i = 0; i < 5; ++i) r[grads[i]] = out[1 + nf + i];
  return r;
}

// Template smoke entries of the reference (gsplat_core/dummy.cpp:7-13).
int dummy_add(int a, int b) { return a + b; }

at::Tensor dummy_array_add(const py::dict& inputs) {
  if (!inputs.contains("a") || !inputs.contains("b"))
    throw std::runtime_error("dummy_array_add input is not an array: a/b");
  return inputs["a"].cast<at::Tensor>() + inputs["b"].cast<at::Tensor>();
}

}  // namespace

// upstream gsplat's selective_adam_update (in place)
void selective_adam_update(at::Tensor param, const at::Tensor& param_grad, at::Tensor exp_avg, at::Tensor exp_avg_sq,
                           const at::Tensor& valid, double lr, double b1, double b2, double eps, int64_t step) {
  gsplat_core::gsplat_selective_adam_update(param, param_grad, exp_avg, exp_avg_sq, valid, lr, b1, b2, eps, step);
}

PYBIND11_MODULE(_gsplat_core, m) {
  m.doc() = "MI355X (gfx950) splatting operator chain with the gsplat_core binding surface.";
  m.def("dummy_add", &dummy_add, py::arg("a"), py::arg("b"));
  m.def("dummy_array_add", &dummy_array_add, py::arg("inputs"));
  m.def("projection_ewa_3dgs_fused_forward", &projection_ewa_3dgs_fused_forward, py::arg("inputs"),
        py::arg("image_width"), py::arg("image_height"), py::arg("eps2d") = 0.3f, py::arg("near_plane") = 0.01f,
        py::arg("far_plane") = 1.0e10f, py::arg("radius_clip") = 0.0f, py::arg("calc_compensations") = false,
        py::arg("camera_model") = 0);
  m.def("projection_ewa_3dgs_fused_backward", &projection_ewa_3dgs_fused_backward, py::arg("inputs"),
        py::arg("forward_outputs"), py::arg("cotangents"), py::arg("image_width"), py::arg("image_height"),
        py::arg("eps2d") = 0.3f, py::arg("camera_model") = 0, py::arg("viewmats_requires_grad") = false);
  m.def("projection_ewa_3dgs_packed_forward", &projection_ewa_3dgs_packed_forward, py::arg("inputs"),
        py::arg("image_width"), py::arg("image_height"), py::arg("eps2d") = 0.3f, py::arg("near_plane") = 0.01f,
        py::arg("far_plane") = 1.0e10f, py::arg("radius_clip") = 0.0f, py::arg("calc_compensations") = false,
        py::arg("camera_model") = 0);
  m.def("projection_ewa_3dgs_packed_backward", &projection_ewa_3dgs_packed_backward, py::arg("inputs"),
        py::arg("forward_outputs"), py::arg("cotangents"), py::arg("image_width"), py::arg("image_height"),
        py::arg("eps2d") = 0.3f, py::arg("camera_model") = 0, py::arg("viewmats_requires_grad") = false);
  m.def("rasterize_to_indices_3dgs_forward", &rasterize_to_indices_3dgs_forward, py::arg("inputs"),
        py::arg("range_start"), py::arg("range_end"), py::arg("image_width"), py::arg("image_height"),
        py::arg("tile_size") = 16);
  m.def("selective_adam_update", &selective_adam_update, py::arg("param"), py::arg("param_grad"),
        py::arg("exp_avg"), py::arg("exp_avg_sq"), py::arg("valid"), py::arg("lr"), py::arg("b1") = 0.9,
        py::arg("b2") = 0.999, py::arg("eps") = 1e-8, py::arg("step") = 0);
  m.def("intersect_tile_forward", &intersect_tile_forward, py::arg("inputs"), py::arg("I"), py::arg("tile_size"),
        py::arg("tile_width"), py::arg("tile_height"), py::arg("sort") = true, py::arg("segmented") = false);
  m.def("intersect_tile_offsets_forward", &intersect_tile_offsets_forward, py::arg("inputs"), py::arg("I"),
        py::arg("tile_size"), py::arg("tile_width"), py::arg("tile_height"));
  py::class_<PendingIntersectHandle>(m, "PendingIntersect");
  m.def("intersect_tile_offsets_begin", &intersect_tile_offsets_begin, py::arg("inputs"), py::arg("I"),
        py::arg("tile_size"), py::arg("tile_width"), py::arg("tile_height"));
  m.def("intersect_tile_offsets_end", &intersect_tile_offsets_end, py::arg("pending"));
  m.def("intersect_offset_forward", &intersect_offset_forward, py::arg("isect_ids"), py::arg("I"),
        py::arg("tile_width"), py::arg("tile_height"));
  m.def("rasterize_to_pixels_3dgs_forward", &rasterize_to_pixels_3dgs_forward, py::arg("inputs"),
        py::arg("image_width"), py::arg("image_height"), py::arg("tile_size"));
  m.def("rasterize_to_pixels_3dgs_backward", &rasterize_to_pixels_3dgs_backward, py::arg("inputs"),
        py::arg("forward_outputs"), py::arg("cotangents"), py::arg("image_width"), py::arg("image_height"),
        py::arg("tile_size"), py::arg("absgrad") = false);
  m.def("spherical_harmonics_forward", &spherical_harmonics_forward, py::arg("degrees_to_use"), py::arg("inputs"));
  m.def("spherical_harmonics_backward", &spherical_harmonics_backward, py::arg("degrees_to_use"), py::arg("inputs"),
        py::arg("cotangents"), py::arg("compute_v_dirs") = true);
  m.def("sh_camera_colors_forward", &sh_camera_colors_forward, py::arg("degrees_to_use"), py::arg("inputs"));
  m.def("sh_camera_colors_packed_forward", &sh_camera_colors_packed_forward, py::arg("degrees_to_use"),
        py::arg("inputs"), py::arg("nnz"));
  m.def("sh_camera_colors_packed_backward", &sh_camera_colors_packed_backward, py::arg("degrees_to_use"),
        py::arg("inputs"), py::arg("cotangents"));
  m.def("sh_camera_colors_backward", &sh_camera_colors_backward, py::arg("degrees_to_use"), py::arg("inputs"),
        py::arg("cotangents"));
  m.def("gaussian_activations_forward", &gaussian_activations_forward, py::arg("inputs"));
  m.def("gaussian_activations_backward", &gaussian_activations_backward, py::arg("inputs"),
        py::arg("forward_outputs"), py::arg("cotangents"));
  m.def("activated_projection_forward", &activated_projection_forward, py::arg("inputs"), py::arg("image_width"),
        py::arg("image_height"), py::arg("eps2d") = 0.3f, py::arg("near_plane") = 0.01f,
        py::arg("far_plane") = 1.0e10f, py::arg("radius_clip") = 0.0f, py::arg("calc_compensations") = false,
        py::arg("camera_model") = 0, py::arg("opacities_in_projection") = false);
  m.def("activated_projection_backward", &activated_projection_backward, py::arg("inputs"),
        py::arg("forward_outputs"), py::arg("cotangents"), py::arg("image_width"), py::arg("image_height"),
        py::arg("eps2d") = 0.3f, py::arg("camera_model") = 0, py::arg("viewmats_requires_grad") = false);
  m.def("activated_projection_packed_forward", &activated_projection_packed_forward, py::arg("inputs"),
        py::arg("image_width"), py::arg("image_height"), py::arg("eps2d") = 0.3f, py::arg("near_plane") = 0.01f,
        py::arg("far_plane") = 1.0e10f, py::arg("radius_clip") = 0.0f, py::arg("calc_compensations") = false,
        py::arg("camera_model") = 0, py::arg("opacities_in_projection") = false);
  m.def("activated_projection_packed_backward", &activated_projection_packed_backward, py::arg("inputs"),
        py::arg("forward_outputs"), py::arg("cotangents"), py::arg("image_width"), py::arg("image_height"),
        py::arg("eps2d") = 0.3f, py::arg("camera_model") = 0, py::arg("viewmats_requires_grad") = false,
        py::arg("viewspace_requires_grad") = false);
  m.def("packed_rows_gather", &packed_rows_gather, py::arg("dense"), py::arg("ids"));
  m.def("packed_rows_scatter", &packed_rows_scatter, py::arg("rows"), py::arg("rank"), py::arg("B"), py::arg("C"),
        py::arg("N"));
  m.def("render_rgb_forward", &render_rgb_forward, py::arg("inputs"), py::arg("image_width"),
        py::arg("image_height"), py::arg("tile_size"), py::arg("eps2d") = 0.3f, py::arg("near_plane") = 0.01f,
        py::arg("far_plane") = 1.0e10f, py::arg("opacities_in_projection") = false, py::arg("accutile") = false);
  m.def("render_rgb_backward", &render_rgb_backward, py::arg("inputs"), py::arg("forward_outputs"),
        py::arg("cotangents"), py::arg("image_width"), py::arg("image_height"), py::arg("tile_size"),
        py::arg("eps2d") = 0.3f, py::arg("accutile") = false, py::arg("viewmats_requires_grad") = false);
  m.def("render_rgb_l1_value_and_grad", &render_rgb_l1_value_and_grad, py::arg("inputs"), py::arg("target"),
        py::arg("image_width"), py::arg("image_height"), py::arg("tile_size"), py::arg("eps2d") = 0.3f,
        py::arg("near_plane") = 0.01f, py::arg("far_plane") = 1.0e10f, py::arg("opacities_in_projection") = false,
        py::arg("accutile") = false);
  m.def("l1_loss_forward", &l1_loss_forward, py::arg("image"), py::arg("target"));
  m.def("l1_loss_backward", &l1_loss_backward, py::arg("image"), py::arg("target"), py::arg("grad"));
  m.def("image_loss_forward", &image_loss_forward, py::arg("image"), py::arg("target"), py::arg("window_size") = 11,
        py::arg("with_maps") = false);
  m.def("image_loss_backward", &image_loss_backward, py::arg("image"), py::arg("target"), py::arg("maps"),
        py::arg("window_size"), py::arg("g_l1"), py::arg("g_ssim"));
  m.def("quat_scale_to_covar_preci_forward", &quat_scale_to_covar_preci_forward, py::arg("inputs"),
        py::arg("compute_covar") = true, py::arg("compute_preci") = true, py::arg("triu") = true);
  m.def("quat_scale_to_covar_preci_backward", &quat_scale_to_covar_preci_backward, py::arg("inputs"),
        py::arg("cotangents"), py::arg("triu") = true);
}
