// Rasterization operator API; mirrors
// gsplat_core/include/gsplat_rasterize.h:12-71 of the reference.
#pragma once

#include "gsplat_common.h"

namespace gsplat_core {

struct RasterizeToPixels3DGSParams {
  int image_width;
  int image_height;
  int tile_size;
  bool use_backgrounds;
  bool use_masks;
  bool packed;
};

struct RasterizeToPixels3DGSInput {
  array means2d;
  array conics;
  array colors;
  array opacities;
  array backgrounds;
  array masks;
  array tile_offsets;
  array flatten_ids;
  StreamOrDevice s;
  RasterizeToPixels3DGSParams params;
};

struct RasterizeToPixels3DGSBackwardInput {
  array means2d;
  array conics;
  array colors;
  array opacities;
  array backgrounds;
  array masks;
  array tile_offsets;
  array flatten_ids;
  array render_alphas;
  array last_ids;
  array v_render_colors;
  array v_render_alphas;
  StreamOrDevice s;
  RasterizeToPixels3DGSParams params;
  bool absgrad;
};

enum RasterizeToPixels3DGSOutputIndex {
  kRenderColors = 0,
  kRenderAlphas = 1,
  kLastIds = 2,
};

enum RasterizeToPixels3DGSBackwardOutputIndex {
  kRasterVMeans2DAbs = 0,
  kRasterVMeans2D = 1,
  kRasterVConics = 2,
  kRasterVColors = 3,
  kRasterVOpacities = 4,
  kRasterVBackgrounds = 5,
};

std::vector<array> gsplat_rasterize_to_pixels_3dgs(const RasterizeToPixels3DGSInput& input);

std::vector<array> gsplat_rasterize_to_pixels_3dgs_backward(const RasterizeToPixels3DGSBackwardInput& input);

// Rasterize to indices (upstream gsplat's rasterize_to_indices_in_range, the
// reference's planned rasterize_to_indices_3dgs_forward): the (flatten id,
// pixel index) pairs the forward composites for list positions
// [range_start, range_end) of each tile, from the given transmittances
// (empty: 1). Returns {gaussian_ids int32 [M], indices int64 [M]}; dense or
// packed Gaussian arrays. Reads the count back to the host (one sync).
std::vector<array> gsplat_rasterize_to_indices_3dgs(int64_t range_start, int64_t range_end, const array& transmittances,
                                                    const array& means2d, const array& conics,
                                                    const array& opacities, int image_width, int image_height,
                                                    int tile_size, const array& tile_offsets,
                                                    const array& flatten_ids, StreamOrDevice s = {});

}  // namespace gsplat_core
