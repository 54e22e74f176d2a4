// The RGB render step in one call per direction (no counterpart operator in
// the reference: its callers compose the operators in Python,
// render_random_3dgs_png.py:61-168 and train_image_fitting_3dgs_mlx.py:
// 165-237). Forward: activated projection, sorted tile intersection with tile
// offsets, rasterization; backward: rasterize VJP, then the activated
// projection's VJP. The operators and their order are those of the composed
// path, so results are the same bit for bit; the Python interpreter is left
// out between them.
#pragma once

#include "gsplat_common.h"

namespace gsplat_core {

struct RenderRGBInput {
  array means;           // [1, N, 3]
  array quats;           // [1, N, 4] raw quaternions
  array log_scales;      // [1, N, 3]
  array opacity_logits;  // [1, N]
  array colors;          // [1, N, ch]
  array viewmats;        // [1, C, 4, 4]
  array Ks;              // [1, C, 3, 3]
  array backgrounds;     // [ch] (one image) or [C, ch]; empty: none
  int image_width = 0;
  int image_height = 0;
  int tile_size = 16;
  float eps2d = 0.3f;
  float near_plane = 0.01f;
  float far_plane = 1e10f;
  bool opacities_in_projection = false;
  bool accutile = false;  // ellipse tile lists
  StreamOrDevice s;
};

enum RenderRGBOutputIndex {
  kRenderRGBColors = 0,      // [1, C, H, W, ch]
  kRenderRGBAlphas = 1,      // [1, C, H, W, 1]
  kRenderRGBLastIds = 2,     // [1, C, H, W]
  kRenderRGBRadii = 3,       // [1, C, N, 2]
  kRenderRGBMeans2D = 4,     // [1, C, N, 2]
  kRenderRGBConics = 5,      // [1, C, N, 3]
  kRenderRGBOpacities = 6,   // [1, C, N] per image (what the rasterizer takes)
  kRenderRGBTilesPerGauss = 7,
  kRenderRGBIsectIds = 8,
  kRenderRGBFlattenIds = 9,
  kRenderRGBTileOffsets = 10,
};

std::vector<array> gsplat_render_rgb_forward(const RenderRGBInput& input);

// {v_means, v_quats, v_log_scales, v_opacity_logits, v_colors, v_viewmats
// (empty unless viewmats_requires_grad)} from the forward's outputs and the
// cotangents of the rendered colours and alphas (empty alphas: zeros).
std::vector<array> gsplat_render_rgb_backward(const RenderRGBInput& input, const std::vector<array>& forward_outputs,
                                              const array& v_render_colors, const array& v_render_alphas,
                                              bool viewmats_requires_grad);

// The step's loss and gradients in one call, as the reference trainer's
// value_and_grad of the L1 image loss (train_image_fitting_3dgs_mlx.py:
// 165-237): the forward above, loss = mean |render_colors - target|, its
// image cotangent (sign(render - target) / count, the L1 backward with
// d loss / d loss = 1) and the backward above. Returns {loss, the forward's
// outputs in RenderRGBOutputIndex order, v_means, v_quats, v_log_scales,
// v_opacity_logits, v_colors}. target: float32, one value per rendered
// colour (viewed as render_colors' shape).
std::vector<array> gsplat_render_rgb_l1_value_and_grad(const RenderRGBInput& input, const array& target);

}  // namespace gsplat_core
