// Fused EWA projection operator layer: validation, output shapes and the
// empty-output conventions follow gsplat_core/gsplat_projection.cpp:67-172,
// 584-652 of the reference; compute is the HIP C-ABI.
#include "gsplat_projection.h"

#include <hip/hip_runtime_api.h>

#include <map>
#include <vector>

#include "core_util.h"
#include "gsplat_training_glue.h"

namespace gsplat_core {
namespace {
using namespace detail;

std::vector<int64_t> projection_shape(const array& means, const array& viewmats, int64_t tail_a,
                                      int64_t tail_b = -1) {
  if (means.dim() < 2 || viewmats.dim() < 3)
    throw std::runtime_error(
        "projection_ewa_3dgs_fused_forward expects means [..., N, 3] and viewmats [..., C, 4, 4].");
  std::vector<int64_t> shape(means.sizes().begin(), means.sizes().end() - 2);
  shape.push_back(viewmats.size(-3));
  shape.push_back(means.size(-2));
  if (tail_a > 0) shape.push_back(tail_a);
  if (tail_b > 0) shape.push_back(tail_b);
  return shape;
}

std::vector<int64_t> projection_scalar_shape(const array& means, const array& viewmats) {
  return projection_shape(means, viewmats, -1);
}

// gsplat_projection.cpp:114-142
void validate_inputs(const ProjectionEWA3DGSFusedInput& in) {
  if (in.means.dim() < 2 || in.means.size(-1) != 3) throw std::runtime_error("means must have shape [..., N, 3].");
  if (in.viewmats.dim() < 3 || in.viewmats.size(-1) != 4 || in.viewmats.size(-2) != 4)
    throw std::runtime_error("viewmats must have shape [..., C, 4, 4].");
  if (in.Ks.dim() < 3 || in.Ks.size(-1) != 3 || in.Ks.size(-2) != 3)
    throw std::runtime_error("Ks must have shape [..., C, 3, 3].");
  if (!in.params.use_covars && (is_empty(in.quats) || is_empty(in.scales)))
    throw std::runtime_error("projection_ewa_3dgs_fused_forward expects covars or quats+scales.");
  if (!is_empty(in.viewspace_points) &&
      in.viewspace_points.sizes().vec() != projection_shape(in.means, in.viewmats, 2))
    throw std::runtime_error("viewspace_points must have shape [..., C, N, 2].");
}

struct Dims {
  int64_t B, C, N;
};

Dims dims_of(const array& means, const array& viewmats, const array& Ks) {
  Dims d;
  d.N = means.size(-2);
  d.C = viewmats.size(-3);
  int64_t b = 1;
  for (int64_t i = 0; i < means.dim() - 2; ++i) b *= means.size(i);
  d.B = b;
  // The kernels index one [4,4] view matrix and one [3,3] K per (batch, camera).
  if (viewmats.numel() != d.B * d.C * 16 || Ks.numel() != d.B * d.C * 9)
    throw std::runtime_error("viewmats and Ks must hold one matrix per (batch, camera) of means' batch prefix.");
  return d;
}

void check_gaussian_params(const array& means, const array& covars, const array& quats, const array& scales,
                           bool use_covars, int64_t BN) {
  require_dtype(means, at::kFloat, "projection_ewa_3dgs_fused expects float32 means.");
  if (use_covars) {
    require_device(covars, "covars");
    require_dtype(covars, at::kFloat, "projection_ewa_3dgs_fused expects float32 covars.");
    if (covars.numel() != BN * 6) throw std::runtime_error("covars must have shape [..., N, 6].");
  } else {
    require_device(quats, "quats");
    require_device(scales, "scales");
    require_dtype(quats, at::kFloat, "projection_ewa_3dgs_fused expects float32 quats.");
    require_dtype(scales, at::kFloat, "projection_ewa_3dgs_fused expects float32 scales.");
    if (quats.numel() != BN * 4 || scales.numel() != BN * 3)
      throw std::runtime_error("quats/scales must have shapes [..., N, 4] / [..., N, 3].");
  }
}

gsplat_projection_params to_c(const ProjectionEWA3DGSFusedParams& p) {
  gsplat_projection_params c;
  c.image_width = p.image_width;
  c.image_height = p.image_height;
  c.eps2d = p.eps2d;
  c.near_plane = p.near_plane;
  c.far_plane = p.far_plane;
  c.radius_clip = p.radius_clip;
  c.calc_compensations = p.calc_compensations;
  c.camera_model = p.camera_model;
  c.use_covars = p.use_covars;
  c.use_opacities = p.use_opacities;
  return c;
}

// The operator (act false) and the activated projection (act true: quats,
// scales and opacities hold raw quaternions, log-scales and opacity logits;
// a sixth output holds the sigmoid opacities).
std::vector<array> projection_forward_impl(const ProjectionEWA3DGSFusedInput& input, bool act) {
  if (act && input.params.use_covars)
    throw std::runtime_error("activated_projection takes quats and log_scales, not covars.");
  validate_inputs(input);
  require_device(input.means, "means");
  require_device(input.viewmats, "viewmats");
  require_device(input.Ks, "Ks");
  const Dims d = dims_of(input.means, input.viewmats, input.Ks);
  const auto& p = input.params;
  check_gaussian_params(input.means, input.covars, input.quats, input.scales, p.use_covars, d.B * d.N);
  const bool have_opac = p.use_opacities || (act && !is_empty(input.opacities));
  if (have_opac) {
    require_device(input.opacities, "opacities");
    require_dtype(input.opacities, at::kFloat, "projection_ewa_3dgs_fused expects float32 opacities.");
    if (input.opacities.numel() != d.B * d.N) throw std::runtime_error("opacities must have shape [..., N].");
  }
  const c10::DeviceGuard guard(input.means.device());
  const array means = contig(input.means);
  const array covars = p.use_covars ? contig(input.covars) : array();
  const array quats = p.use_covars ? array() : contig(input.quats);
  const array scales = p.use_covars ? array() : contig(input.scales);
  const array opac = have_opac ? contig(input.opacities) : array();
  const array viewmats = contig(input.viewmats.to(at::kFloat));
  const array Ks = contig(input.Ks.to(at::kFloat));
  const auto scalar_shape = projection_scalar_shape(means, viewmats);
  array means2d = at::empty(projection_shape(means, viewmats, 2), f32_like(means));
  array depths = at::empty(scalar_shape, f32_like(means));
  array conics = at::empty(projection_shape(means, viewmats, 3), f32_like(means));
  array comps = p.calc_compensations ? at::empty(scalar_shape, f32_like(means)) : at::empty({0}, f32_like(means));
  array radii = at::empty(projection_shape(means, viewmats, 2), i32_like(means));
  const gsplat_projection_params cp = to_c(p);
  if (!act) {
    check(gsplat_hip_projection_fwd(means.data_ptr<float>(), p.use_covars ? covars.data_ptr<float>() : nullptr,
                                    p.use_covars ? nullptr : quats.data_ptr<float>(),
                                    p.use_covars ? nullptr : scales.data_ptr<float>(),
                                    p.use_opacities ? opac.data_ptr<float>() : nullptr, viewmats.data_ptr<float>(),
                                    Ks.data_ptr<float>(), d.B, d.C, d.N, &cp, radii.data_ptr<int32_t>(),
                                    means2d.data_ptr<float>(), depths.data_ptr<float>(), conics.data_ptr<float>(),
                                    p.calc_compensations ? comps.data_ptr<float>() : nullptr,
                                    stream_for(input.s, means)));
    return {means2d, depths, conics, comps, radii};
  }
  array opac_out = have_opac ? at::empty(opac.sizes(), f32_like(means)) : at::empty({0}, f32_like(means));
  check(gsplat_hip_activated_projection_fwd(
      means.data_ptr<float>(), quats.data_ptr<float>(), scales.data_ptr<float>(),
      have_opac ? opac.data_ptr<float>() : nullptr, viewmats.data_ptr<float>(), Ks.data_ptr<float>(), d.B, d.C,
      d.N, &cp, radii.data_ptr<int32_t>(), means2d.data_ptr<float>(), depths.data_ptr<float>(),
      conics.data_ptr<float>(), p.calc_compensations ? comps.data_ptr<float>() : nullptr,
      have_opac ? opac_out.data_ptr<float>() : nullptr, stream_for(input.s, means)));
  return {means2d, depths, conics, comps, radii, opac_out};
}

// The operator (act false) and the activated projection (act true; logits and
// v_opac feed the fifth output, the opacity logits' gradient).
std::vector<array> projection_backward_impl(const ProjectionEWA3DGSFusedBackwardInput& input, bool act,
                                            const array& logits_in, const array& v_opac_in) {
  if (act && input.params.use_covars)
    throw std::runtime_error("activated_projection takes quats and log_scales, not covars.");
  // gsplat_projection.cpp:144-172
  ProjectionEWA3DGSFusedInput fwd;
  fwd.means = input.means;
  fwd.covars = input.covars;
  fwd.quats = input.quats;
  fwd.scales = input.scales;
  fwd.viewmats = input.viewmats;
  fwd.Ks = input.Ks;
  fwd.params = input.params;
  validate_inputs(fwd);
  if (input.params.camera_model < 0 || input.params.camera_model > 2)
    throw std::runtime_error("projection_ewa_3dgs_fused_backward: unknown camera model.");
  if (input.radii.scalar_type() != at::kInt) throw std::runtime_error("radii must be int32.");
  // an empty v_depths stands for zeros (callers whose loss ignores depths)
  const bool use_v_depths = !is_empty(input.v_depths);
  if (input.v_means2d.sizes().vec() != projection_shape(input.means, input.viewmats, 2) ||
      input.v_conics.sizes().vec() != projection_shape(input.means, input.viewmats, 3) ||
      (use_v_depths && input.v_depths.sizes().vec() != projection_scalar_shape(input.means, input.viewmats)))
    throw std::runtime_error("projection backward cotangent shape mismatch.");
  require_device(input.means, "means");
  require_device(input.viewmats, "viewmats");
  require_device(input.Ks, "Ks");
  const Dims d = dims_of(input.means, input.viewmats, input.Ks);
  const auto& p = input.params;
  check_gaussian_params(input.means, input.covars, input.quats, input.scales, p.use_covars, d.B * d.N);
  const int64_t BCN = d.B * d.C * d.N;
  if (input.radii.numel() != BCN * 2 || input.conics.numel() != BCN * 3)
    throw std::runtime_error("radii / conics must have shapes [..., C, N, 2] / [..., C, N, 3].");
  const bool use_comp = p.calc_compensations && !is_empty(input.compensations) && !is_empty(input.v_compensations);
  if (use_comp && (input.compensations.numel() != BCN || input.v_compensations.numel() != BCN))
    throw std::runtime_error("compensations / v_compensations must have shape [..., C, N].");
  const c10::DeviceGuard guard(input.means.device());
  const array means = contig(input.means);
  const array covars = p.use_covars ? contig(input.covars) : array();
  const array quats = p.use_covars ? array() : contig(input.quats);
  const array scales = p.use_covars ? array() : contig(input.scales);
  const array viewmats = contig(input.viewmats.to(at::kFloat));
  const array Ks = contig(input.Ks.to(at::kFloat));
  const array radii = contig(input.radii);
  const array conics = contig(input.conics.to(at::kFloat));
  const array comps = use_comp ? contig(input.compensations.to(at::kFloat)) : array();
  const array v_comps = use_comp ? contig(input.v_compensations.to(at::kFloat)) : array();
  const array v_m2 = contig(input.v_means2d.to(at::kFloat));
  const array v_dep = use_v_depths ? contig(input.v_depths.to(at::kFloat)) : array();
  const array v_con = contig(input.v_conics.to(at::kFloat));
  array v_means = at::empty(means.sizes(), f32_like(means));
  array v_covars = p.use_covars ? at::empty(covars.sizes(), f32_like(means)) : at::empty({0}, f32_like(means));
  array v_quats = p.use_covars ? at::empty({0}, f32_like(means)) : at::empty(quats.sizes(), f32_like(means));
  array v_scales = p.use_covars ? at::empty({0}, f32_like(means)) : at::empty(scales.sizes(), f32_like(means));
  array v_viewmats = input.viewmats_requires_grad ? at::empty(viewmats.sizes(), f32_like(means))
                                                  : at::empty({0}, f32_like(means));
  const size_t ws_bytes =
      gsplat_hip_projection_bwd_workspace_size(d.B, d.C, d.N, input.viewmats_requires_grad ? 1 : 0);
  array ws = at::empty({static_cast<int64_t>(ws_bytes)}, u8_like(means));
  const gsplat_projection_params cp = to_c(p);
  if (act) {
    const bool have_logits = !is_empty(logits_in);
    const bool have_v_opac = have_logits && !is_empty(v_opac_in);
    if (have_logits) {
      require_device(logits_in, "opacity_logits");
      require_dtype(logits_in, at::kFloat, "activated_projection expects float32 opacity_logits.");
      if (logits_in.numel() != d.B * d.N) throw std::runtime_error("opacity_logits must have shape [..., N].");
    }
    if (have_v_opac) {
      require_device(v_opac_in, "v_opacities");
      if (v_opac_in.numel() != d.B * d.N) throw std::runtime_error("v_opacities must have shape [..., N].");
    }
    const array logits = have_logits ? contig(logits_in) : array();
    const array v_opac = have_v_opac ? contig(v_opac_in.to(at::kFloat)) : array();
    array v_logits = have_logits ? at::empty(logits.sizes(), f32_like(means)) : at::empty({0}, f32_like(means));
    check(gsplat_hip_activated_projection_bwd(
        means.data_ptr<float>(), quats.data_ptr<float>(), scales.data_ptr<float>(),
        have_logits ? logits.data_ptr<float>() : nullptr, viewmats.data_ptr<float>(), Ks.data_ptr<float>(), d.B,
        d.C, d.N, &cp, radii.data_ptr<int32_t>(), conics.data_ptr<float>(),
        use_comp ? comps.data_ptr<float>() : nullptr, v_m2.data_ptr<float>(),
        use_v_depths ? v_dep.data_ptr<float>() : nullptr, v_con.data_ptr<float>(),
        use_comp ? v_comps.data_ptr<float>() : nullptr, have_v_opac ? v_opac.data_ptr<float>() : nullptr,
        v_means.data_ptr<float>(), v_quats.data_ptr<float>(), v_scales.data_ptr<float>(),
        have_logits ? v_logits.data_ptr<float>() : nullptr,
        input.viewmats_requires_grad ? v_viewmats.data_ptr<float>() : nullptr,
        ws_bytes ? ws.data_ptr<uint8_t>() : nullptr, ws_bytes, stream_for(input.s, means)));
    return {v_means, v_quats, v_scales, v_logits, v_viewmats};
  }
  check(gsplat_hip_projection_bwd(
      means.data_ptr<float>(), p.use_covars ? covars.data_ptr<float>() : nullptr,
      p.use_covars ? nullptr : quats.data_ptr<float>(), p.use_covars ? nullptr : scales.data_ptr<float>(),
      viewmats.data_ptr<float>(), Ks.data_ptr<float>(), d.B, d.C, d.N, &cp, radii.data_ptr<int32_t>(),
      conics.data_ptr<float>(), use_comp ? comps.data_ptr<float>() : nullptr, v_m2.data_ptr<float>(),
      use_v_depths ? v_dep.data_ptr<float>() : nullptr, v_con.data_ptr<float>(),
      use_comp ? v_comps.data_ptr<float>() : nullptr,
      v_means.data_ptr<float>(), p.use_covars ? v_covars.data_ptr<float>() : nullptr,
      p.use_covars ? nullptr : v_quats.data_ptr<float>(), p.use_covars ? nullptr : v_scales.data_ptr<float>(),
      input.viewmats_requires_grad ? v_viewmats.data_ptr<float>() : nullptr,
      ws_bytes ? ws.data_ptr<uint8_t>() : nullptr, ws_bytes, stream_for(input.s, means)));
  return {v_means, v_covars, v_quats, v_scales, v_viewmats};
}

// The packed count, read on the kernels' stream.
int64_t read_count(const array& dev_count, void* stream) {
  int64_t host = 0;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t err = hipMemcpyAsync(&host, dev_count.data_ptr<int64_t>(), sizeof(int64_t), hipMemcpyDeviceToHost, s);
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  if (err != hipSuccess)
    throw std::runtime_error(std::string("projection_ewa_3dgs_packed_forward: reading the count failed: ") +
                             hipGetErrorString(err));
  if (host > static_cast<int64_t>(INT32_MAX))
    throw std::runtime_error("projection_ewa_3dgs_packed_forward: more than 2^31-1 visible pairs.");
  return host;
}

// int32 copy of caller ids (upstream passes int64).
array ids32(const array& a, const char* name) {
  require_device(a, name);
  if (a.scalar_type() != at::kInt && a.scalar_type() != at::kLong)
    throw std::runtime_error(std::string(name) + " must be int32 or int64.");
  return contig(a.to(at::kInt));
}

}  // namespace

std::vector<array> gsplat_projection_ewa_3dgs_packed(const ProjectionEWA3DGSFusedInput& input) {
  validate_inputs(input);
  require_device(input.means, "means");
  require_device(input.viewmats, "viewmats");
  require_device(input.Ks, "Ks");
  const Dims d = dims_of(input.means, input.viewmats, input.Ks);
  const auto& p = input.params;
  check_gaussian_params(input.means, input.covars, input.quats, input.scales, p.use_covars, d.B * d.N);
  if (p.use_opacities) {
    require_device(input.opacities, "opacities");
    require_dtype(input.opacities, at::kFloat, "projection_ewa_3dgs_packed expects float32 opacities.");
    if (input.opacities.numel() != d.B * d.N) throw std::runtime_error("opacities must have shape [..., N].");
  }
  const c10::DeviceGuard guard(input.means.device());
  const array means = contig(input.means);
  const array covars = p.use_covars ? contig(input.covars) : array();
  const array quats = p.use_covars ? array() : contig(input.quats);
  const array scales = p.use_covars ? array() : contig(input.scales);
  const array opac = p.use_opacities ? contig(input.opacities) : array();
  const array viewmats = contig(input.viewmats.to(at::kFloat));
  const array Ks = contig(input.Ks.to(at::kFloat));
  void* stream = stream_for(input.s, means);
  const gsplat_projection_params cp = to_c(p);
  const size_t ws_bytes = gsplat_hip_projection_packed_workspace_size(d.B, d.C, d.N, 0);
  array ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, u8_like(means));
  array count = at::empty({1}, i64_like(means));
  const float* cov_p = p.use_covars ? covars.data_ptr<float>() : nullptr;
  const float* q_p = p.use_covars ? nullptr : quats.data_ptr<float>();
  const float* s_p = p.use_covars ? nullptr : scales.data_ptr<float>();
  const float* o_p = p.use_opacities ? opac.data_ptr<float>() : nullptr;
  check(gsplat_hip_projection_packed_count(means.data_ptr<float>(), cov_p, q_p, s_p, o_p, viewmats.data_ptr<float>(),
                                           Ks.data_ptr<float>(), d.B, d.C, d.N, &cp, count.data_ptr<int64_t>(),
                                           ws.data_ptr<uint8_t>(), ws_bytes, stream));
  const int64_t nnz = d.B * d.C * d.N > 0 ? read_count(count, stream) : 0;
  auto i32 = [&](std::vector<int64_t> shape) { return at::empty(shape, i32_like(means)); };
  auto f32 = [&](std::vector<int64_t> shape) { return at::empty(shape, f32_like(means)); };
  array batch_ids = i32({nnz}), camera_ids = i32({nnz}), gaussian_ids = i32({nnz});
  array indptr = i32({d.B * d.C + 1});
  array radii = i32({nnz, 2});
  array means2d = f32({nnz, 2}), depths = f32({nnz}), conics = f32({nnz, 3});
  array comps = p.calc_compensations ? f32({nnz}) : f32({0});
  check(gsplat_hip_projection_packed_fwd(
      means.data_ptr<float>(), cov_p, q_p, s_p, o_p, viewmats.data_ptr<float>(), Ks.data_ptr<float>(), d.B, d.C, d.N,
      &cp, nnz, batch_ids.data_ptr<int32_t>(), camera_ids.data_ptr<int32_t>(), gaussian_ids.data_ptr<int32_t>(),
      indptr.data_ptr<int32_t>(), radii.data_ptr<int32_t>(), means2d.data_ptr<float>(), depths.data_ptr<float>(),
      conics.data_ptr<float>(), p.calc_compensations ? comps.data_ptr<float>() : nullptr, ws.data_ptr<uint8_t>(),
      ws_bytes, stream));
  return {batch_ids, camera_ids, gaussian_ids, indptr, radii, means2d, depths, conics, comps};
}

std::vector<array> gsplat_projection_ewa_3dgs_packed_backward(const ProjectionEWA3DGSPackedBackwardInput& input) {
  ProjectionEWA3DGSFusedInput fwd;
  fwd.means = input.means;
  fwd.covars = input.covars;
  fwd.quats = input.quats;
  fwd.scales = input.scales;
  fwd.viewmats = input.viewmats;
  fwd.Ks = input.Ks;
  fwd.params = input.params;
  validate_inputs(fwd);
  if (input.params.camera_model < 0 || input.params.camera_model > 2)
    throw std::runtime_error("projection_ewa_3dgs_packed_backward: unknown camera model.");
  require_device(input.means, "means");
  require_device(input.viewmats, "viewmats");
  require_device(input.Ks, "Ks");
  const Dims d = dims_of(input.means, input.viewmats, input.Ks);
  const auto& p = input.params;
  check_gaussian_params(input.means, input.covars, input.quats, input.scales, p.use_covars, d.B * d.N);
  const int64_t nnz = input.camera_ids.numel();
  const bool use_v_depths = !is_empty(input.v_depths);
  if (input.gaussian_ids.numel() != nnz || (!is_empty(input.batch_ids) && input.batch_ids.numel() != nnz) ||
      input.conics.numel() != nnz * 3 || input.v_means2d.numel() != nnz * 2 || input.v_conics.numel() != nnz * 3 ||
      (use_v_depths && input.v_depths.numel() != nnz))
    throw std::runtime_error("projection_ewa_3dgs_packed_backward: packed inputs must have nnz rows.");
  if (d.B > 1 && is_empty(input.batch_ids))
    throw std::runtime_error("projection_ewa_3dgs_packed_backward: batch_ids are needed with more than one batch.");
  const bool use_comp = p.calc_compensations && !is_empty(input.compensations) && !is_empty(input.v_compensations);
  if (use_comp && (input.compensations.numel() != nnz || input.v_compensations.numel() != nnz))
    throw std::runtime_error("compensations / v_compensations must have nnz rows.");
  const c10::DeviceGuard guard(input.means.device());
  const array means = contig(input.means);
  const array covars = p.use_covars ? contig(input.covars) : array();
  const array quats = p.use_covars ? array() : contig(input.quats);
  const array scales = p.use_covars ? array() : contig(input.scales);
  const array viewmats = contig(input.viewmats.to(at::kFloat));
  const array Ks = contig(input.Ks.to(at::kFloat));
  const array bid = is_empty(input.batch_ids) ? array() : ids32(input.batch_ids, "batch_ids");
  const array cid = ids32(input.camera_ids, "camera_ids");
  const array gid = ids32(input.gaussian_ids, "gaussian_ids");
  const array conics = contig(input.conics.to(at::kFloat));
  const array comps = use_comp ? contig(input.compensations.to(at::kFloat)) : array();
  const array v_comps = use_comp ? contig(input.v_compensations.to(at::kFloat)) : array();
  const array v_m2 = contig(input.v_means2d.to(at::kFloat));
  const array v_dep = use_v_depths ? contig(input.v_depths.to(at::kFloat)) : array();
  const array v_con = contig(input.v_conics.to(at::kFloat));
  array v_means = at::empty(means.sizes(), f32_like(means));
  array v_covars = p.use_covars ? at::empty(covars.sizes(), f32_like(means)) : at::empty({0}, f32_like(means));
  array v_quats = p.use_covars ? at::empty({0}, f32_like(means)) : at::empty(quats.sizes(), f32_like(means));
  array v_scales = p.use_covars ? at::empty({0}, f32_like(means)) : at::empty(scales.sizes(), f32_like(means));
  array v_viewmats = input.viewmats_requires_grad ? at::empty(viewmats.sizes(), f32_like(means))
                                                  : at::empty({0}, f32_like(means));
  const size_t ws_bytes =
      gsplat_hip_projection_packed_workspace_size(d.B, d.C, d.N, input.viewmats_requires_grad ? 1 : 0);
  array ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, u8_like(means));
  const gsplat_projection_params cp = to_c(p);
  check(gsplat_hip_projection_packed_bwd(
      means.data_ptr<float>(), p.use_covars ? covars.data_ptr<float>() : nullptr,
      p.use_covars ? nullptr : quats.data_ptr<float>(), p.use_covars ? nullptr : scales.data_ptr<float>(),
      viewmats.data_ptr<float>(), Ks.data_ptr<float>(), d.B, d.C, d.N, &cp, nnz,
      is_empty(bid) ? nullptr : bid.data_ptr<int32_t>(), cid.data_ptr<int32_t>(), gid.data_ptr<int32_t>(),
      conics.data_ptr<float>(), use_comp ? comps.data_ptr<float>() : nullptr, v_m2.data_ptr<float>(),
      use_v_depths ? v_dep.data_ptr<float>() : nullptr, v_con.data_ptr<float>(),
      use_comp ? v_comps.data_ptr<float>() : nullptr, v_means.data_ptr<float>(),
      p.use_covars ? v_covars.data_ptr<float>() : nullptr, p.use_covars ? nullptr : v_quats.data_ptr<float>(),
      p.use_covars ? nullptr : v_scales.data_ptr<float>(),
      input.viewmats_requires_grad ? v_viewmats.data_ptr<float>() : nullptr, ws.data_ptr<uint8_t>(), ws_bytes,
      stream_for(input.s, means)));
  return {v_means, v_covars, v_quats, v_scales, v_viewmats};
}

namespace {

// Speculative packed forward: a call whose shape (device, B, C, N) was seen
// before writes its rows into outputs sized by the previous count plus an
// eighth, queued behind the count pass before the count reaches the host
// (the kernels bound every write by that capacity and take indptr's total
// from the device). The rows are then narrowed to the count; a count over
// the capacity runs the forward again into exact outputs. Hints are per host
// thread.
int64_t& packed_hint(int64_t B, int64_t C, int64_t N) {
  thread_local std::map<std::vector<int64_t>, int64_t> hints;
  int dev = 0;
  (void)hipGetDevice(&dev);
  return hints[{dev, B, C, N}];
}

}  // namespace

std::vector<array> gsplat_activated_projection_packed_forward(const ProjectionEWA3DGSFusedInput& input) {
  const char* op = "activated_projection_packed_forward";
  if (input.params.use_covars) throw std::runtime_error(std::string(op) + " takes quats and log_scales, not covars.");
  validate_inputs(input);
  require_device(input.means, "means");
  require_device(input.viewmats, "viewmats");
  require_device(input.Ks, "Ks");
  const Dims d = dims_of(input.means, input.viewmats, input.Ks);
  const auto& p = input.params;
  check_gaussian_params(input.means, input.covars, input.quats, input.scales, false, d.B * d.N);
  const bool have_logits = !is_empty(input.opacities);
  if (p.use_opacities && !have_logits) throw std::runtime_error(std::string(op) + ": use_opacities without logits.");
  if (have_logits) {
    require_device(input.opacities, "opacity_logits");
    require_dtype(input.opacities, at::kFloat, "activated_projection_packed expects float32 opacity_logits.");
    if (input.opacities.numel() != d.B * d.N) throw std::runtime_error("opacity_logits must have shape [..., N].");
  }
  const c10::DeviceGuard guard(input.means.device());
  const array means = contig(input.means);
  const array quats = contig(input.quats);
  const array scales = contig(input.scales);
  const array logits = have_logits ? contig(input.opacities) : array();
  const array viewmats = contig(input.viewmats.to(at::kFloat));
  const array Ks = contig(input.Ks.to(at::kFloat));
  void* stream = stream_for(input.s, means);
  const gsplat_projection_params cp = to_c(p);
  const size_t ws_bytes = gsplat_hip_projection_packed_workspace_size(d.B, d.C, d.N, 0);
  array ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, u8_like(means));
  array count = at::empty({1}, i64_like(means));
  const float* l_p = have_logits ? logits.data_ptr<float>() : nullptr;
  check(gsplat_hip_activated_projection_packed_count(means.data_ptr<float>(), quats.data_ptr<float>(),
                                                     scales.data_ptr<float>(), l_p, viewmats.data_ptr<float>(),
                                                     Ks.data_ptr<float>(), d.B, d.C, d.N, &cp,
                                                     count.data_ptr<int64_t>(), ws.data_ptr<uint8_t>(), ws_bytes,
                                                     stream));
  auto i32 = [&](std::vector<int64_t> shape) { return at::empty(shape, i32_like(means)); };
  auto f32 = [&](std::vector<int64_t> shape) { return at::empty(shape, f32_like(means)); };
  array indptr = i32({d.B * d.C + 1});
  // rows of `rows` capacity; nnz_dev: the count on the device (speculative)
  auto run = [&](int64_t rows, const int64_t* nnz_dev) {
    std::vector<array> o = {i32({rows}),    i32({rows}),    i32({rows}),
                            indptr,         i32({rows, 2}), f32({rows, 2}),
                            f32({rows}),    f32({rows, 3}), p.calc_compensations ? f32({rows}) : f32({0}),
                            have_logits ? f32({rows}) : f32({0})};
    check(gsplat_hip_activated_projection_packed_fwd(
        means.data_ptr<float>(), quats.data_ptr<float>(), scales.data_ptr<float>(), l_p, viewmats.data_ptr<float>(),
        Ks.data_ptr<float>(), d.B, d.C, d.N, &cp, rows, nnz_dev, o[0].data_ptr<int32_t>(), o[1].data_ptr<int32_t>(),
        o[2].data_ptr<int32_t>(), indptr.data_ptr<int32_t>(), o[4].data_ptr<int32_t>(), o[5].data_ptr<float>(),
        o[6].data_ptr<float>(), o[7].data_ptr<float>(), p.calc_compensations ? o[8].data_ptr<float>() : nullptr,
        have_logits ? o[9].data_ptr<float>() : nullptr, ws.data_ptr<uint8_t>(), ws_bytes, stream));
    return o;
  };
  if (d.B * d.C * d.N == 0) {
    auto o = run(0, nullptr);
    o.push_back(ws);
    return o;
  }
  int64_t& hint = packed_hint(d.B, d.C, d.N);
  std::vector<array> out;
  int64_t nnz = -1;
  if (hint > 0) {
    const int64_t cap = std::min(d.B * d.C * d.N, hint + hint / 8 + 1024);
    out = run(cap, count.data_ptr<int64_t>());
    nnz = read_count(count, stream);
    if (nnz <= cap) {
      for (size_t i = 0; i < out.size(); ++i)
        if (i != 3 && out[i].numel() > 0) out[i] = out[i].narrow(0, 0, nnz);
    } else {
      out.clear();
    }
  }
  if (out.empty()) {
    if (nnz < 0) nnz = read_count(count, stream);
    out = run(nnz, nullptr);
  }
  hint = nnz;
  out.push_back(ws);
  return out;
}

std::vector<array> gsplat_activated_projection_packed_backward(const ProjectionEWA3DGSPackedBackwardInput& input,
                                                               const array& rank, const array& opacity_logits,
                                                               const array& v_opacities, bool viewspace_grad) {
  const char* op = "activated_projection_packed_backward";
  if (input.params.use_covars) throw std::runtime_error(std::string(op) + " takes quats and log_scales, not covars.");
  ProjectionEWA3DGSFusedInput fwd;
  fwd.means = input.means;
  fwd.quats = input.quats;
  fwd.scales = input.scales;
  fwd.viewmats = input.viewmats;
  fwd.Ks = input.Ks;
  fwd.params = input.params;
  validate_inputs(fwd);
  if (input.params.camera_model < 0 || input.params.camera_model > 2)
    throw std::runtime_error(std::string(op) + ": unknown camera model.");
  require_device(input.means, "means");
  require_device(input.viewmats, "viewmats");
  require_device(input.Ks, "Ks");
  const Dims d = dims_of(input.means, input.viewmats, input.Ks);
  const auto& p = input.params;
  check_gaussian_params(input.means, input.covars, input.quats, input.scales, false, d.B * d.N);
  const int64_t nnz = input.conics.numel() / 3;
  const bool use_v_depths = !is_empty(input.v_depths);
  const bool have_logits = !is_empty(opacity_logits);
  const bool have_v_opac = have_logits && !is_empty(v_opacities);
  if (input.conics.numel() != nnz * 3 || input.v_means2d.numel() != nnz * 2 || input.v_conics.numel() != nnz * 3 ||
      (use_v_depths && input.v_depths.numel() != nnz) || (have_v_opac && v_opacities.numel() != nnz))
    throw std::runtime_error(std::string(op) + ": packed inputs must have nnz rows.");
  const size_t rank_bytes = gsplat_hip_projection_packed_workspace_size(d.B, d.C, d.N, 0);
  require_device(rank, "rank");
  if (rank.scalar_type() != at::kByte || static_cast<size_t>(rank.numel()) < rank_bytes)
    throw std::runtime_error(std::string(op) + ": rank must be the forward's uint8 workspace.");
  const bool use_comp = p.calc_compensations && !is_empty(input.compensations) && !is_empty(input.v_compensations);
  if (use_comp && (input.compensations.numel() != nnz || input.v_compensations.numel() != nnz))
    throw std::runtime_error("compensations / v_compensations must have nnz rows.");
  if (have_logits) {
    require_device(opacity_logits, "opacity_logits");
    require_dtype(opacity_logits, at::kFloat, "activated_projection_packed expects float32 opacity_logits.");
    if (opacity_logits.numel() != d.B * d.N) throw std::runtime_error("opacity_logits must have shape [..., N].");
  }
  const c10::DeviceGuard guard(input.means.device());
  const array means = contig(input.means);
  const array quats = contig(input.quats);
  const array scales = contig(input.scales);
  const array viewmats = contig(input.viewmats.to(at::kFloat));
  const array Ks = contig(input.Ks.to(at::kFloat));
  const array conics = contig(input.conics.to(at::kFloat));
  const array comps = use_comp ? contig(input.compensations.to(at::kFloat)) : array();
  const array v_comps = use_comp ? contig(input.v_compensations.to(at::kFloat)) : array();
  const array v_m2 = contig(input.v_means2d.to(at::kFloat));
  const array v_dep = use_v_depths ? contig(input.v_depths.to(at::kFloat)) : array();
  const array v_con = contig(input.v_conics.to(at::kFloat));
  const array logits = have_logits ? contig(opacity_logits) : array();
  const array v_opac = have_v_opac ? contig(v_opacities.to(at::kFloat)) : array();
  const array rk = contig(rank);
  array v_means = at::empty(means.sizes(), f32_like(means));
  array v_quats = at::empty(quats.sizes(), f32_like(means));
  array v_scales = at::empty(scales.sizes(), f32_like(means));
  array v_logits = have_logits ? at::empty(logits.sizes(), f32_like(means)) : at::empty({0}, f32_like(means));
  array v_viewmats = input.viewmats_requires_grad ? at::empty(viewmats.sizes(), f32_like(means))
                                                  : at::empty({0}, f32_like(means));
  array v_viewspace = viewspace_grad ? at::empty(projection_shape(means, viewmats, 2), f32_like(means))
                                     : at::empty({0}, f32_like(means));
  const size_t ws_bytes =
      gsplat_hip_projection_packed_workspace_size(d.B, d.C, d.N, input.viewmats_requires_grad ? 1 : 0);
  array ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, u8_like(means));
  const gsplat_projection_params cp = to_c(p);
  check(gsplat_hip_activated_projection_packed_bwd(
      means.data_ptr<float>(), quats.data_ptr<float>(), scales.data_ptr<float>(),
      have_logits ? logits.data_ptr<float>() : nullptr, viewmats.data_ptr<float>(), Ks.data_ptr<float>(), d.B, d.C,
      d.N, &cp, nnz, rk.data_ptr<uint8_t>(), static_cast<size_t>(rk.numel()), conics.data_ptr<float>(),
      use_comp ? comps.data_ptr<float>() : nullptr, v_m2.data_ptr<float>(),
      use_v_depths ? v_dep.data_ptr<float>() : nullptr, v_con.data_ptr<float>(),
      use_comp ? v_comps.data_ptr<float>() : nullptr, have_v_opac ? v_opac.data_ptr<float>() : nullptr,
      v_means.data_ptr<float>(), v_quats.data_ptr<float>(), v_scales.data_ptr<float>(),
      have_logits ? v_logits.data_ptr<float>() : nullptr,
      input.viewmats_requires_grad ? v_viewmats.data_ptr<float>() : nullptr,
      viewspace_grad ? v_viewspace.data_ptr<float>() : nullptr, ws.data_ptr<uint8_t>(), ws_bytes,
      stream_for(input.s, means)));
  return {v_means, v_quats, v_scales, v_logits, v_viewmats, v_viewspace};
}

array gsplat_packed_rows_gather(const array& dense, const array& batch_ids, const array& camera_ids,
                                const array& gaussian_ids, StreamOrDevice s) {
  require_device(dense, "dense");
  require_dtype(dense, at::kFloat, "packed_rows_gather expects float32 values.");
  if (dense.dim() != 4) throw std::runtime_error("packed_rows_gather: dense must have shape [B, C, N, K].");
  const int64_t B = dense.size(0), C = dense.size(1), N = dense.size(2), K = dense.size(3);
  const int64_t nnz = camera_ids.numel();
  if (gaussian_ids.numel() != nnz || (!is_empty(batch_ids) && batch_ids.numel() != nnz))
    throw std::runtime_error("packed_rows_gather: ids must have nnz entries.");
  if (B > 1 && is_empty(batch_ids)) throw std::runtime_error("packed_rows_gather: batch_ids needed with B > 1.");
  const c10::DeviceGuard guard(dense.device());
  const array d = contig(dense);
  const array bid = is_empty(batch_ids) ? array() : ids32(batch_ids, "batch_ids");
  const array cid = ids32(camera_ids, "camera_ids");
  const array gid = ids32(gaussian_ids, "gaussian_ids");
  array rows = at::empty({nnz, K}, f32_like(d));
  check(gsplat_hip_packed_rows_gather(d.data_ptr<float>(), is_empty(bid) ? nullptr : bid.data_ptr<int32_t>(),
                                      cid.data_ptr<int32_t>(), gid.data_ptr<int32_t>(), nnz, B, C, N,
                                      static_cast<int32_t>(K), rows.data_ptr<float>(), stream_for(s, d)));
  return rows;
}

array gsplat_packed_rows_scatter(const array& rows, const array& rank, int64_t B, int64_t C, int64_t N,
                                 StreamOrDevice s) {
  require_device(rows, "rows");
  require_dtype(rows, at::kFloat, "packed_rows_scatter expects float32 values.");
  if (rows.dim() != 2) throw std::runtime_error("packed_rows_scatter: rows must have shape [nnz, K].");
  require_device(rank, "rank");
  if (rank.scalar_type() != at::kByte) throw std::runtime_error("packed_rows_scatter: rank must be uint8.");
  const int64_t nnz = rows.size(0), K = rows.size(1);
  const c10::DeviceGuard guard(rows.device());
  const array r = contig(rows);
  const array rk = contig(rank);
  array dense = at::empty({B, C, N, K}, f32_like(r));
  check(gsplat_hip_packed_rows_scatter(r.data_ptr<float>(), rk.data_ptr<uint8_t>(), static_cast<size_t>(rk.numel()),
                                       nnz, B, C, N, static_cast<int32_t>(K), dense.data_ptr<float>(),
                                       stream_for(s, r)));
  return dense;
}

std::vector<array> gsplat_projection_ewa_3dgs_fused(const ProjectionEWA3DGSFusedInput& input) {
  return projection_forward_impl(input, false);
}

std::vector<array> gsplat_projection_ewa_3dgs_fused_backward(const ProjectionEWA3DGSFusedBackwardInput& input) {
  return projection_backward_impl(input, false, array(), array());
}

std::vector<array> gsplat_activated_projection_forward(const ProjectionEWA3DGSFusedInput& input) {
  return projection_forward_impl(input, true);
}

std::vector<array> gsplat_activated_projection_backward(const ProjectionEWA3DGSFusedBackwardInput& input,
                                                        const array& opacity_logits, const array& v_opacities) {
  return projection_backward_impl(input, true, opacity_logits, v_opacities);
}

}  // namespace gsplat_core
