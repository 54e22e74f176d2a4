// Training-step glue around the operator chain (no counterpart operator in
// the reference: these replace its framework elementwise composition at the
// call sites, scanner_points_training_utils.py:39-41, 306-316 and the image
// loss of image_loss_components, :1123-1172).
#pragma once

#include "gsplat_common.h"
#include "gsplat_projection.h"

namespace gsplat_core {

// Activated projection: the activations below fused into the fused EWA
// projection. The fields of `input` carry the raw model parameters: quats
// (quaternions), scales (log-scales) and opacities (opacity logits, may be
// empty); params.use_covars must be false. Returns the projection's
// {means2d, depths, conics, compensations, radii} plus opacities =
// sigmoid(opacity_logits) (empty without logits), equal to
// gsplat_gaussian_activations_forward followed by the projection.
std::vector<array> gsplat_activated_projection_forward(const ProjectionEWA3DGSFusedInput& input);

// {v_means, v_quats, v_log_scales, v_opacity_logits, v_viewmats}: the
// projection's VJP through the activations; `input` as the projection
// backward's with raw quats and log-scales, plus the opacity logits and the
// cotangent of the opacities output (empty: zeros).
std::vector<array> gsplat_activated_projection_backward(const ProjectionEWA3DGSFusedBackwardInput& input,
                                                        const array& opacity_logits, const array& v_opacities);

// Activated packed projection: the activations fused into the packed
// projection (gsplat_projection_ewa_3dgs_packed), fields as
// gsplat_activated_projection_forward's. Returns {batch_ids, camera_ids,
// gaussian_ids, indptr, radii, means2d, depths, conics, compensations,
// opacities, rank}: the packed rows, each row's sigmoid opacity (empty
// without logits) and the uint8 rank structure the backward reads.
std::vector<array> gsplat_activated_projection_packed_forward(const ProjectionEWA3DGSFusedInput& input);

// {v_means, v_quats, v_log_scales, v_opacity_logits, v_viewmats,
// v_viewspace} of the activated packed projection: `input` as the packed
// backward's with raw quats and log-scales (the ids are not read), the
// forward's rank, the opacity logits and the per-row cotangent of the
// opacities (empty: zeros). v_viewspace ([..., C, N, 2], empty unless
// viewspace_grad): the means2d rows' cotangent at their dense (camera,
// Gaussian) slots, zeros elsewhere -- the gradient of a dense viewspace
// proxy.
std::vector<array> gsplat_activated_projection_packed_backward(const ProjectionEWA3DGSPackedBackwardInput& input,
                                                               const array& rank, const array& opacity_logits,
                                                               const array& v_opacities, bool viewspace_grad = false);

// Packed rows [nnz, K] of dense [B, C, N, K] values at the rows' (batch,
// camera, Gaussian) ids (batch_ids may be empty with B = 1).
array gsplat_packed_rows_gather(const array& dense, const array& batch_ids, const array& camera_ids,
                                const array& gaussian_ids, StreamOrDevice s = {});

// Its adjoint: dense [B, C, N, K] holding each row at its pair's slot (the
// activated packed forward's rank) and zeros elsewhere.
array gsplat_packed_rows_scatter(const array& rows, const array& rank, int64_t B, int64_t C, int64_t N,
                                 StreamOrDevice s = {});

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

// Image loss terms of image_loss_components (scanner_points_training_utils.py:
// 1123-1172) for image and target [B, H, W, C] float32 (NHWC, the layout of
// the reference's conv2d): {values, maps} with values [2] = {mean|image -
// target|, ssim_index(image, target, window_size)}. maps [3, B, Ho, Wo, C]
// (with_maps; else empty) holds the per-window derivatives the backward
// reads (Ho = H + 2 (window / 2) - window + 1, Wo likewise).
std::vector<array> gsplat_image_loss_forward(const array& image, const array& target, int window_size,
                                             bool with_maps, StreamOrDevice s = {});

// v_image for the 0-d device cotangents g_l1 of the L1 value and g_ssim of
// the SSIM value (either may be empty: zero); maps from the forward (may be
// empty when g_ssim is). The target gets no gradient.
array gsplat_image_loss_backward(const array& image, const array& target, const array& maps, int window_size,
                                 const array& g_l1, const array& g_ssim, StreamOrDevice s = {});

// Selective Adam step in place (upstream gsplat's selective_adam_update): the
// rows (first dimension) of param with valid != 0 (valid empty: all) take
// torch.optim.Adam's step number `step` (step <= 0: no bias correction, as
// upstream's kernel); the other rows and their moments are unchanged.
void gsplat_selective_adam_update(array& param, const array& grad, array& exp_avg, array& exp_avg_sq,
                                  const array& valid, double lr, double b1, double b2, double eps, int64_t step,
                                  StreamOrDevice s = {});

}  // namespace gsplat_core
