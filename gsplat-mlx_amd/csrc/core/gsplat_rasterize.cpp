// Rasterization operator layer: validation and output shapes follow
// gsplat_core/gsplat_rasterize.cpp:44-247 of the reference; compute is the
// HIP C-ABI.
#include "gsplat_rasterize.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>

#include "core_util.h"

namespace gsplat_core {
namespace {
using namespace detail;

// gsplat_rasterize.cpp:44-88
// Packed layout (params.packed, rejected by the reference at :48-51): the
// Gaussian arrays have nnz rows that flatten_ids index directly.
void validate_rasterize_input(const RasterizeToPixels3DGSInput& in) {
  if (in.params.packed) {
    if (in.means2d.dim() != 2 || in.means2d.size(-1) != 2) throw std::runtime_error("means2d must have shape [nnz, 2].");
    const int64_t nnz = in.means2d.size(0);
    if (in.conics.dim() != 2 || in.conics.size(0) != nnz || in.conics.size(1) != 3)
      throw std::runtime_error("conics must have shape [nnz, 3].");
    if (in.colors.dim() != 2 || in.colors.size(0) != nnz) throw std::runtime_error("colors must have shape [nnz, channels].");
    if (in.opacities.dim() != 1 || in.opacities.size(0) != nnz) throw std::runtime_error("opacities must have shape [nnz].");
    if (in.tile_offsets.dim() < 3)
      throw std::runtime_error("tile_offsets must have shape [..., tile_height, tile_width].");
    if (in.flatten_ids.dim() != 1) throw std::runtime_error("flatten_ids must have shape [n_isects].");
    if (in.params.use_masks && in.masks.sizes() != in.tile_offsets.sizes())
      throw std::runtime_error("masks must have the same shape as tile_offsets.");
    return;
  }
  if (in.means2d.dim() < 3 || in.means2d.size(-1) != 2) throw std::runtime_error("means2d must have shape [..., N, 2].");
  if (in.conics.dim() != in.means2d.dim() || in.conics.size(-1) != 3)
    throw std::runtime_error("conics must have shape [..., N, 3].");
  if (in.colors.dim() != in.means2d.dim() || in.colors.size(-2) != in.means2d.size(-2))
    throw std::runtime_error("colors must have shape [..., N, channels].");
  if (in.opacities.dim() + 1 != in.means2d.dim()) throw std::runtime_error("opacities must have shape [..., N].");
  if (in.tile_offsets.dim() < 3)
    throw std::runtime_error("tile_offsets must have shape [..., tile_height, tile_width].");
  if (in.flatten_ids.dim() != 1) throw std::runtime_error("flatten_ids must have shape [n_isects].");
  if (in.params.use_masks && in.masks.sizes() != in.tile_offsets.sizes())
    throw std::runtime_error("masks must have the same shape as tile_offsets.");
}

std::vector<int64_t> image_prefix(const array& tile_offsets) {
  return std::vector<int64_t>(tile_offsets.sizes().begin(), tile_offsets.sizes().end() - 2);
}

struct Layout {
  int64_t I, N;
  int channels, th, tw;
};

Layout layout_of(const RasterizeToPixels3DGSInput& in) {
  Layout l;
  l.N = in.means2d.size(-2);
  l.channels = static_cast<int>(in.colors.size(-1));
  l.th = static_cast<int>(in.tile_offsets.size(-2));
  l.tw = static_cast<int>(in.tile_offsets.size(-1));
  l.I = (l.th * l.tw) ? in.tile_offsets.numel() / (static_cast<int64_t>(l.th) * l.tw) : 0;
  if (in.params.packed) {  // N = nnz rows, shapes checked by validate_rasterize_input
    if (in.params.use_backgrounds && in.backgrounds.numel() != l.I * l.channels)
      throw std::runtime_error("backgrounds must have shape [..., channels].");
    return l;
  }
  if (in.means2d.numel() / 2 != l.I * l.N)
    throw std::runtime_error(
        "rasterize_to_pixels_3dgs dense path expects means2d size to equal I * N * 2.");
  if (in.conics.numel() != l.I * l.N * 3 || in.colors.numel() != l.I * l.N * l.channels ||
      in.opacities.numel() != l.I * l.N)
    throw std::runtime_error("rasterize_to_pixels_3dgs: conics/colors/opacities do not match means2d.");
  if (in.params.use_backgrounds && in.backgrounds.numel() != l.I * l.channels)
    throw std::runtime_error("backgrounds must have shape [..., channels].");
  return l;
}

void require_inputs(const RasterizeToPixels3DGSInput& in) {
  require_device(in.means2d, "means2d");
  require_device(in.conics, "conics");
  require_device(in.colors, "colors");
  require_device(in.opacities, "opacities");
  require_device(in.tile_offsets, "tile_offsets");
  require_device(in.flatten_ids, "flatten_ids");
  if (in.params.use_backgrounds) require_device(in.backgrounds, "backgrounds");
  if (in.params.use_masks) require_device(in.masks, "masks");
  for (const array* a : {&in.means2d, &in.conics, &in.colors, &in.opacities})
    require_dtype(*a, at::kFloat, "rasterize_to_pixels_3dgs expects float32 means2d/conics/colors/opacities.");
  require_dtype(in.tile_offsets, at::kInt, "tile_offsets must be int32.");
  require_dtype(in.flatten_ids, at::kInt, "flatten_ids must be int32.");
}

}  // namespace

std::vector<array> gsplat_rasterize_to_pixels_3dgs(const RasterizeToPixels3DGSInput& input) {
  validate_rasterize_input(input);
  require_inputs(input);
  const Layout l = layout_of(input);
  const auto& p = input.params;
  const c10::DeviceGuard guard(input.means2d.device());
  const array means2d = contig(input.means2d), conics = contig(input.conics), colors = contig(input.colors);
  const array opac = contig(input.opacities), offsets = contig(input.tile_offsets), flat = contig(input.flatten_ids);
  const array bg = p.use_backgrounds ? contig(input.backgrounds.to(at::kFloat)) : array();
  const array masks = p.use_masks ? mask_u8(input.masks) : array();
  auto prefix = image_prefix(offsets);
  auto rc_shape = prefix, ra_shape = prefix, li_shape = prefix;
  rc_shape.insert(rc_shape.end(), {p.image_height, p.image_width, l.channels});
  ra_shape.insert(ra_shape.end(), {p.image_height, p.image_width, 1});
  li_shape.insert(li_shape.end(), {p.image_height, p.image_width});
  array render_colors = at::empty(rc_shape, f32_like(means2d));
  array render_alphas = at::empty(ra_shape, f32_like(means2d));
  array last_ids = at::empty(li_shape, i32_like(means2d));
  check((p.packed ? gsplat_hip_rasterize_fwd_packed : gsplat_hip_rasterize_fwd)(
                                 means2d.data_ptr<float>(), conics.data_ptr<float>(), colors.data_ptr<float>(),
                                 opac.data_ptr<float>(), p.use_backgrounds ? bg.data_ptr<float>() : nullptr,
                                 p.use_masks ? masks.data_ptr<uint8_t>() : nullptr, offsets.data_ptr<int32_t>(),
                                 flat.data_ptr<int32_t>(), l.I, l.N, l.channels, p.image_width, p.image_height,
                                 p.tile_size, l.tw, l.th, flat.numel(), render_colors.data_ptr<float>(),
                                 render_alphas.data_ptr<float>(), last_ids.data_ptr<int32_t>(),
                                 stream_for(input.s, means2d)));
  return {render_colors, render_alphas, last_ids};
}

std::vector<array> gsplat_rasterize_to_pixels_3dgs_backward(const RasterizeToPixels3DGSBackwardInput& input) {
  RasterizeToPixels3DGSInput fwd;
  fwd.means2d = input.means2d;
  fwd.conics = input.conics;
  fwd.colors = input.colors;
  fwd.opacities = input.opacities;
  fwd.backgrounds = input.backgrounds;
  fwd.masks = input.masks;
  fwd.tile_offsets = input.tile_offsets;
  fwd.flatten_ids = input.flatten_ids;
  fwd.params = input.params;
  validate_rasterize_input(fwd);
  // gsplat_rasterize.cpp:104-122
  if (input.render_alphas.dim() < 3 || input.render_alphas.size(-1) != 1)
    throw std::runtime_error("render_alphas must have shape [..., H, W, 1].");
  if (input.last_ids.dim() + 1 != input.render_alphas.dim())
    throw std::runtime_error("last_ids must have shape [..., H, W].");
  const auto& p = input.params;
  auto rc_shape = image_prefix(input.tile_offsets);
  rc_shape.insert(rc_shape.end(), {p.image_height, p.image_width, input.colors.size(-1)});
  if (input.v_render_colors.sizes().vec() != rc_shape) throw std::runtime_error("v_render_colors shape mismatch.");
  // an empty v_render_alphas stands for zeros (losses on the colours only)
  const bool use_v_ra = !is_empty(input.v_render_alphas);
  if (use_v_ra && input.v_render_alphas.sizes() != input.render_alphas.sizes())
    throw std::runtime_error("v_render_alphas shape mismatch.");
  require_inputs(fwd);
  const Layout l = layout_of(fwd);
  const int64_t n_pix = l.I * p.image_height * p.image_width;
  if (input.render_alphas.numel() != n_pix || input.last_ids.numel() != n_pix)
    throw std::runtime_error("render_alphas / last_ids do not match the image size.");
  require_device(input.render_alphas, "render_alphas");
  require_device(input.last_ids, "last_ids");
  require_device(input.v_render_colors, "v_render_colors");
  if (use_v_ra) require_device(input.v_render_alphas, "v_render_alphas");
  require_dtype(input.last_ids, at::kInt, "last_ids must be int32.");
  const c10::DeviceGuard guard(input.means2d.device());
  const array means2d = contig(input.means2d), conics = contig(input.conics), colors = contig(input.colors);
  const array opac = contig(input.opacities), offsets = contig(input.tile_offsets), flat = contig(input.flatten_ids);
  const array bg = p.use_backgrounds ? contig(input.backgrounds.to(at::kFloat)) : array();
  const array masks = p.use_masks ? mask_u8(input.masks) : array();
  const array ra = contig(input.render_alphas.to(at::kFloat)), li = contig(input.last_ids);
  const array v_rc = contig(input.v_render_colors.to(at::kFloat));
  const array v_ra = use_v_ra ? contig(input.v_render_alphas.to(at::kFloat)) : array();
  array v_abs = input.absgrad ? at::empty(means2d.sizes(), f32_like(means2d)) : at::empty({0}, f32_like(means2d));
  array v_m2 = at::empty(means2d.sizes(), f32_like(means2d));
  array v_con = at::empty(conics.sizes(), f32_like(means2d));
  array v_col = at::empty(colors.sizes(), f32_like(means2d));
  array v_op = at::empty(opac.sizes(), f32_like(means2d));
  array v_bg = p.use_backgrounds ? at::empty(bg.sizes(), f32_like(means2d)) : at::empty({0}, f32_like(means2d));
  const size_t ws_bytes = gsplat_hip_rasterize_bwd_workspace_size(l.I, static_cast<int32_t>(l.channels), l.tw, l.th);
  array ws = at::empty({static_cast<int64_t>(std::max<size_t>(ws_bytes, 1))}, u8_like(means2d));
  check((p.packed ? gsplat_hip_rasterize_bwd_packed : gsplat_hip_rasterize_bwd)(
      means2d.data_ptr<float>(), conics.data_ptr<float>(), colors.data_ptr<float>(), opac.data_ptr<float>(),
      p.use_backgrounds ? bg.data_ptr<float>() : nullptr, p.use_masks ? masks.data_ptr<uint8_t>() : nullptr,
      offsets.data_ptr<int32_t>(), flat.data_ptr<int32_t>(), l.I, l.N, l.channels, p.image_width, p.image_height,
      p.tile_size, l.tw, l.th, flat.numel(), ra.data_ptr<float>(), li.data_ptr<int32_t>(), v_rc.data_ptr<float>(),
      use_v_ra ? v_ra.data_ptr<float>() : nullptr, input.absgrad ? v_abs.data_ptr<float>() : nullptr,
      v_m2.data_ptr<float>(),
      v_con.data_ptr<float>(), v_col.data_ptr<float>(), v_op.data_ptr<float>(),
      p.use_backgrounds ? v_bg.data_ptr<float>() : nullptr, ws.data_ptr<uint8_t>(), ws_bytes,
      stream_for(input.s, means2d)));
  return {v_abs, v_m2, v_con, v_col, v_op, v_bg};
}

std::vector<array> gsplat_rasterize_to_indices_3dgs(int64_t range_start, int64_t range_end, const array& transmittances,
                                                    const array& means2d_in, const array& conics_in,
                                                    const array& opacities_in, int image_width, int image_height,
                                                    int tile_size, const array& tile_offsets_in,
                                                    const array& flatten_ids_in, StreamOrDevice s) {
  for (const auto* a : {&means2d_in, &conics_in, &opacities_in, &tile_offsets_in, &flatten_ids_in})
    require_device(*a, "rasterize_to_indices_3dgs input");
  for (const array* a : {&means2d_in, &conics_in, &opacities_in})
    require_dtype(*a, at::kFloat, "rasterize_to_indices_3dgs expects float32 means2d/conics/opacities.");
  require_dtype(tile_offsets_in, at::kInt, "tile_offsets must be int32.");
  require_dtype(flatten_ids_in, at::kInt, "flatten_ids must be int32.");
  if (tile_offsets_in.dim() < 3) throw std::runtime_error("tile_offsets must have shape [..., tile_height, tile_width].");
  if (means2d_in.size(-1) != 2 || conics_in.numel() != means2d_in.numel() / 2 * 3 ||
      opacities_in.numel() != means2d_in.numel() / 2)
    throw std::runtime_error("rasterize_to_indices_3dgs: means2d/conics/opacities shapes do not match.");
  const int th = static_cast<int>(tile_offsets_in.size(-2)), tw = static_cast<int>(tile_offsets_in.size(-1));
  const int64_t I = th * tw ? tile_offsets_in.numel() / (static_cast<int64_t>(th) * tw) : 0;
  const int64_t n_pix = I * image_width * static_cast<int64_t>(image_height);
  const bool use_t = !is_empty(transmittances);
  if (use_t) {
    require_device(transmittances, "transmittances");
    if (transmittances.numel() != n_pix)
      throw std::runtime_error("transmittances must have shape [..., image_height, image_width].");
  }
  const c10::DeviceGuard guard(means2d_in.device());
  const array means2d = contig(means2d_in), conics = contig(conics_in), opac = contig(opacities_in);
  const array offsets = contig(tile_offsets_in), flat = contig(flatten_ids_in);
  const array trans = use_t ? contig(transmittances.to(at::kFloat)) : array();
  void* stream = stream_for(s, means2d);
  const int64_t n_rows = means2d.numel() / 2;
  array starts = at::empty({std::max<int64_t>(n_pix, 1)}, i32_like(means2d));
  array total = at::empty({1}, i64_like(means2d));
  const size_t ws_bytes = gsplat_hip_rasterize_to_indices_workspace_size(I, image_width, image_height);
  array ws = at::empty({static_cast<int64_t>(std::max<size_t>(ws_bytes, 1))}, u8_like(means2d));
  const float* tp = use_t ? trans.data_ptr<float>() : nullptr;
  check(gsplat_hip_rasterize_to_indices_count(range_start, range_end, tp, means2d.data_ptr<float>(),
                                              conics.data_ptr<float>(), opac.data_ptr<float>(),
                                              offsets.data_ptr<int32_t>(), flat.data_ptr<int32_t>(), I, n_rows,
                                              image_width, image_height, tile_size, tw, th, flat.numel(),
                                              starts.data_ptr<int32_t>(), total.data_ptr<int64_t>(),
                                              ws.data_ptr<uint8_t>(), ws_bytes, stream));
  int64_t m = 0;
  const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  hipError_t err = hipMemcpyAsync(&m, total.data_ptr<int64_t>(), sizeof(int64_t), hipMemcpyDeviceToHost, hs);
  if (err == hipSuccess) err = hipStreamSynchronize(hs);
  if (err != hipSuccess)
    throw std::runtime_error(std::string("rasterize_to_indices_3dgs: reading the count failed: ") +
                             hipGetErrorString(err));
  if (m > static_cast<int64_t>(INT32_MAX)) throw std::runtime_error("rasterize_to_indices_3dgs: more than 2^31-1 entries.");
  array gids = at::empty({m}, i32_like(means2d));
  array idx = at::empty({m}, i64_like(means2d));
  check(gsplat_hip_rasterize_to_indices_write(range_start, range_end, tp, means2d.data_ptr<float>(),
                                              conics.data_ptr<float>(), opac.data_ptr<float>(),
                                              offsets.data_ptr<int32_t>(), flat.data_ptr<int32_t>(), I, n_rows,
                                              image_width, image_height, tile_size, tw, th, flat.numel(),
                                              starts.data_ptr<int32_t>(), m, m ? gids.data_ptr<int32_t>() : nullptr,
                                              m ? idx.data_ptr<int64_t>() : nullptr, stream));
  return {gids, idx};
}

}  // namespace gsplat_core
