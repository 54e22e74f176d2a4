// Training-step glue around the operator chain (no counterpart operator in
// the reference: these replace its framework elementwise composition at the
// call sites, scanner_points_training_utils.py:39-41, 306-316 and the L1 term
// of image_loss_components, :1147-1160).
#pragma once

#include "gsplat_common.h"

namespace gsplat_core {

// {quats / max(|quats|, 1e-8), exp(log_scales), sigmoid(opacity_logits)};
// each input may be undefined / empty (its output is then empty).
std::vector<array> gsplat_gaussian_activations_forward(const array& quats, const array& log_scales,
                                                       const array& opacity_logits, StreamOrDevice s = {});

// {v_quats, v_log_scales, v_opacity_logits} from the cotangents of the three
// outputs (an empty cotangent counts as zero); reads the raw quats and the
// forward's scales and opacities.
std::vector<array> gsplat_gaussian_activations_backward(const array& quats, const array& scales,
                                                        const array& opacities, const array& v_quats_out,
                                                        const array& v_scales, const array& v_opacities,
                                                        StreamOrDevice s = {});

// mean(|a - b|) as a 0-d device tensor.
array gsplat_l1_loss_forward(const array& a, const array& b, StreamOrDevice s = {});

// {v_a, v_b} = {g / n * sign(a - b), -(g / n) * sign(a - b)} for the 0-d
// device cotangent g.
std::vector<array> gsplat_l1_loss_backward(const array& a, const array& b, const array& grad, StreamOrDevice s = {});

}  // namespace gsplat_core
