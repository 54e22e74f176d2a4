// The RGB render step in one call per direction: the operators of the
// composed path (activated projection, sorted tile intersection with offsets,
// rasterization, and their VJPs in reverse), called from C++ in the same
// order with the same inputs.
#include "gsplat_render.h"

#include <map>
#include <mutex>

#include "core_util.h"
#include "gsplat_intersect.h"
#include "gsplat_projection.h"
#include "gsplat_rasterize.h"
#include "gsplat_training_glue.h"

namespace gsplat_core {
namespace {
using namespace detail;

int64_t n_cameras(const RenderRGBInput& in) {
  if (in.viewmats.dim() < 3) throw std::runtime_error("render_rgb: viewmats must have shape [..., C, 4, 4].");
  return in.viewmats.size(-3);
}

// [1, N, ...] per Gaussian -> [1, C, N, ...] per image: a view for one
// camera, else an expanded contiguous copy (what the composed path builds).
array per_image(const array& a, int64_t C) {
  const array v = a.unsqueeze(1);
  if (C == 1) return v;
  std::vector<int64_t> shape = v.sizes().vec();
  shape[1] = C;
  return v.expand(shape).contiguous();
}

// The sum over images of a per-image gradient, shaped like the per-Gaussian
// input (the expand's VJP).
array sum_images(const array& g, int64_t C, const array& like) {
  if (C == 1) return g.reshape(like.sizes());
  return g.sum(1).reshape(like.sizes());
}

RasterizeToPixels3DGSParams raster_params(const RenderRGBInput& in) {
  return {in.image_width, in.image_height, in.tile_size, !is_empty(in.backgrounds), false, false};
}

void validate(const RenderRGBInput& in) {
  for (const array* a : {&in.means, &in.quats, &in.log_scales, &in.opacity_logits, &in.colors, &in.viewmats, &in.Ks})
    if (is_empty(*a)) throw std::runtime_error("render_rgb: means, quats, log_scales, opacity_logits, colors, "
                                               "viewmats and Ks are required.");
  if (in.means.dim() != 3 || in.means.size(0) != 1)
    throw std::runtime_error("render_rgb: means must have shape [1, N, 3].");
  if (in.colors.dim() != 3 || in.colors.size(1) != in.means.size(1))
    throw std::runtime_error("render_rgb: colors must have shape [1, N, channels].");
  if (in.tile_size <= 0 || in.image_width <= 0 || in.image_height <= 0)
    throw std::runtime_error("render_rgb: invalid image or tile size.");
}

}  // namespace

std::vector<array> gsplat_render_rgb_forward(const RenderRGBInput& in) {
  validate(in);
  const int64_t C = n_cameras(in);
  ProjectionEWA3DGSFusedInput p;
  p.means = in.means;
  p.quats = in.quats;
  p.scales = in.log_scales;
  p.opacities = in.opacity_logits;
  p.viewmats = in.viewmats;
  p.Ks = in.Ks;
  p.s = in.s;
  p.params = {in.image_width, in.image_height, in.eps2d, in.near_plane, in.far_plane, 0.0f, false, 0, false,
              in.opacities_in_projection};
  const auto proj = gsplat_activated_projection_forward(p);
  const array opac_img = per_image(proj[5], C);

  IntersectTileInput it;
  it.means2d = proj[kMeans2D];
  it.radii = proj[kRadii];
  it.depths = proj[kDepths];
  it.conics = in.accutile ? proj[kConics] : empty_f32();
  it.opacities = in.accutile ? opac_img : empty_f32();
  it.image_ids = empty_f32();
  it.gaussian_ids = empty_f32();
  it.s = in.s;
  const int tw = (in.image_width + in.tile_size - 1) / in.tile_size;
  const int th = (in.image_height + in.tile_size - 1) / in.tile_size;
  it.params = {static_cast<int>(C), in.tile_size, tw, th, true, false, false, in.accutile, in.accutile};
  const auto isect = gsplat_intersect_tile_with_offsets(it);

  RasterizeToPixels3DGSInput r;
  r.means2d = proj[kMeans2D];
  r.conics = proj[kConics];
  r.colors = per_image(in.colors, C);
  r.opacities = opac_img;
  r.backgrounds = is_empty(in.backgrounds) ? empty_f32() : in.backgrounds;
  r.masks = empty_f32();
  r.tile_offsets = isect[3];
  r.flatten_ids = isect[kFlattenIds];
  r.s = in.s;
  r.params = raster_params(in);
  const auto img = gsplat_rasterize_to_pixels_3dgs(r);
  return {img[kRenderColors], img[kRenderAlphas], img[kLastIds], proj[kRadii], proj[kMeans2D], proj[kConics],
          opac_img, isect[kTilesPerGauss], isect[kIsectIds], isect[kFlattenIds], isect[3]};
}

std::vector<array> gsplat_render_rgb_backward(const RenderRGBInput& in, const std::vector<array>& fwd,
                                              const array& v_render_colors, const array& v_render_alphas,
                                              bool viewmats_requires_grad) {
  validate(in);
  if (fwd.size() < kRenderRGBTileOffsets + 1) throw std::runtime_error("render_rgb_backward: missing forward outputs.");
  const int64_t C = n_cameras(in);
  RasterizeToPixels3DGSBackwardInput rb;
  rb.means2d = fwd[kRenderRGBMeans2D];
  rb.conics = fwd[kRenderRGBConics];
  rb.colors = per_image(in.colors, C);
  rb.opacities = fwd[kRenderRGBOpacities];
  rb.backgrounds = is_empty(in.backgrounds) ? empty_f32() : in.backgrounds;
  rb.masks = empty_f32();
  rb.tile_offsets = fwd[kRenderRGBTileOffsets];
  rb.flatten_ids = fwd[kRenderRGBFlattenIds];
  rb.render_alphas = fwd[kRenderRGBAlphas];
  rb.last_ids = fwd[kRenderRGBLastIds];
  rb.v_render_colors = contig(v_render_colors);
  rb.v_render_alphas = is_empty(v_render_alphas) ? empty_f32() : contig(v_render_alphas);
  rb.s = in.s;
  rb.params = raster_params(in);
  rb.absgrad = false;
  const auto g = gsplat_rasterize_to_pixels_3dgs_backward(rb);

  ProjectionEWA3DGSFusedBackwardInput pb;
  pb.means = in.means;
  pb.quats = in.quats;
  pb.scales = in.log_scales;
  pb.viewmats = in.viewmats;
  pb.Ks = in.Ks;
  pb.radii = fwd[kRenderRGBRadii];
  pb.conics = fwd[kRenderRGBConics];
  pb.compensations = empty_f32();
  pb.v_means2d = contig(g[kRasterVMeans2D]);
  pb.v_depths = empty_f32();
  pb.v_conics = contig(g[kRasterVConics]);
  pb.v_compensations = empty_f32();
  pb.s = in.s;
  pb.params = {in.image_width, in.image_height, in.eps2d, -1.0e20f, 1.0e20f, 0.0f, false, 0, false, false};
  pb.viewmats_requires_grad = viewmats_requires_grad;
  const array v_opac = contig(sum_images(g[kRasterVOpacities], C, in.opacity_logits));
  const auto pg = gsplat_activated_projection_backward(pb, in.opacity_logits, v_opac);
  return {pg[0], pg[1], pg[2], pg[3], sum_images(g[kRasterVColors], C, in.colors),
          viewmats_requires_grad ? pg[4] : empty_f32()};
}

namespace {

// A device scalar 1.0 (the loss's own cotangent) per device, created once
// and never written. The map is never destroyed: its tensors must not be
// freed at process exit, after the device runtime may have shut down.
const array& device_one(const array& like) {
  static std::mutex mu;
  static auto* ones = new std::map<int, array>();
  const std::lock_guard<std::mutex> lock(mu);
  const int dev = like.device().index();
  auto it = ones->find(dev);
  if (it == ones->end()) it = ones->emplace(dev, at::ones({}, f32_like(like))).first;
  return it->second;
}

}  // namespace

std::vector<array> gsplat_render_rgb_l1_value_and_grad(const RenderRGBInput& in, const array& target_in) {
  std::vector<array> fwd = gsplat_render_rgb_forward(in);
  const array& image = fwd[kRenderRGBColors];
  if (target_in.scalar_type() != at::kFloat || target_in.numel() != image.numel() ||
      target_in.device() != image.device())
    throw std::runtime_error("render_rgb_l1_value_and_grad: target must be float32 with one value per rendered "
                             "colour, on the render's device.");
  const c10::DeviceGuard guard(image.device());
  const array target = contig(target_in).view(image.sizes());
  array loss = gsplat_l1_loss_forward(image, target, in.s);
  // d loss / d image with d loss / d loss = 1; no target gradient
  array v_image = at::empty(image.sizes(), f32_like(image));
  if (image.numel() > 0)
    check(gsplat_hip_l1_loss_bwd(image.data_ptr<float>(), target.data_ptr<float>(), image.numel(),
                                 device_one(image).data_ptr<float>(), v_image.data_ptr<float>(), nullptr,
                                 stream_for(in.s, image)));
  std::vector<array> grads = gsplat_render_rgb_backward(in, fwd, v_image, array(), false);
  std::vector<array> out;
  out.reserve(1 + fwd.size() + 5);
  out.push_back(loss);
  out.insert(out.end(), fwd.begin(), fwd.end());
  out.insert(out.end(), grads.begin(), grads.begin() + 5);
  return out;
}

}  // namespace gsplat_core
