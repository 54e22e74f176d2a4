// Fused EWA projection (forward / backward) for gfx950.
//
// Forward: one lane per (camera, Gaussian); blockIdx.y selects the camera so
// viewmat and K are wave-uniform (scalar loads). Culling follows the
// reference GPU kernel (gsplat_core/metal/gsplat_projection.metal:214-339);
// per-Gaussian math follows gsplat_core/gsplat_projection.cpp:446-521 in the
// same operation order (file compiled without FMA contraction).
//
// Backward (projection_bwd.hip, compiled for gradients with FMA contraction
// and fast division): one lane per (batch, Gaussian) looping over the C
// cameras (no atomics), as gsplat_projection.metal:446-569. The view-matrix gradient is a
// sum over Gaussians per camera: each block reduces its lanes' 12 partials
// with wave DPP sums + LDS and writes one row of a partials buffer, which a
// second kernel sums per camera (deterministic; replaces the reference's
// one-thread-per-camera O(N) loop, gsplat_projection.metal:571-676).
//
// Activated projection (ACT = true): the same kernels read the model's raw
// parameters -- quaternions, log-scales and opacity logits -- and apply the
// training step's activations (quats / max(|quats|, 1e-8), exp, sigmoid;
// scanner_points_training_utils.py:39-41, 306-316) on load, with the
// operations of training_glue.hip's activation kernels, so the result equals
// the activation kernel followed by the projection bit for bit. The forward
// also writes the sigmoid opacities the rasterizer takes; the backward maps
// the quaternion and scale gradients through the activations and turns the
// rasterizer's opacity gradient into the logits' gradient.
#include "projection_common.hpp"

namespace gsplat_hip {
namespace {

// ACT: quats, scales and opacities hold the raw parameters (quaternions,
// log-scales, opacity logits) and opac_out (if non-null) receives the sigmoid
// opacities, written by the first camera of each batch.
template <bool ACT>
__global__ void __launch_bounds__(kProjBlock) projection_fwd_kernel(
    const float* __restrict__ means, const float* __restrict__ covars, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ opacities, const float* __restrict__ viewmats,
    const float* __restrict__ Ks, int64_t C, int64_t N, gsplat_projection_params p, int32_t* __restrict__ radii,
    float* __restrict__ means2d, float* __restrict__ depths, float* __restrict__ conics,
    float* __restrict__ compensations, float* __restrict__ opac_out) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kProjBlock + threadIdx.x;
  if (n >= N) return;
  const int64_t cam = blockIdx.y;  // b * C + c
  const int64_t b = cam / C;
  const int64_t g = b * N + n;
  const int64_t idx = cam * N + n;
  const CamFrame f = load_camera(viewmats + cam * 16, Ks + cam * 9);
  if constexpr (ACT) {
    if (opac_out && cam == b * C) opac_out[g] = sigmoid_of(opacities[g]);
  }

  int32_t rx_out = 0, ry_out = 0;
  float m2x = 0.0f, m2y = 0.0f, depth = 0.0f, c0 = 0.0f, c1 = 0.0f, c2 = 0.0f, comp_out = 0.0f;

  const float mw[3] = {means[g * 3], means[g * 3 + 1], means[g * 3 + 2]};
  float mc[3];
  world_to_cam(f, mw, mc);
  bool valid = !(mc[2] < p.near_plane || mc[2] > p.far_plane);
  if (valid) {
    Mat3 cw;
    if (p.use_covars) {
      cw = read_covar(covars + g * 6);
    } else {
      float q[4], s[3];
      load_quat_scale<ACT>(quats, scales, g, q, s);
      cw = covar_from_quat_scale(q, s);
    }
    const Mat3 cc = mat3_mul(mat3_mul(f.R, cw), mat3_tr(f.R));
    float J[6], m2[2];
    camera_jacobian(p.camera_model, mc, f, p.image_width, p.image_height, J, m2);
    float cov2d[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int row = 0; row < 2; ++row)
#pragma unroll
      for (int col = 0; col < 2; ++col) {
        float acc = 0.0f;
#pragma unroll
        for (int a = 0; a < 3; ++a)
#pragma unroll
          for (int bb = 0; bb < 3; ++bb) acc += J[row * 3 + a] * cc.v[a * 3 + bb] * J[col * 3 + bb];
        cov2d[row * 2 + col] = acc;
      }
    const float det_orig = cov2d[0] * cov2d[3] - cov2d[1] * cov2d[2];
    cov2d[0] += p.eps2d;
    cov2d[3] += p.eps2d;
    const float det = cov2d[0] * cov2d[3] - cov2d[1] * cov2d[2];
    const float comp = sqrtf(fmaxf(kMinCompensation * kMinCompensation, det_orig / det));
    valid = det > 0.0f;
    float extend = kGaussianExtend;
    if (valid && p.use_opacities) {
      float op = ACT ? sigmoid_of(opacities[g]) : opacities[g];
      if (p.calc_compensations) op *= comp;
      valid = !(op < kAlphaThreshold);
      if (valid) extend = fminf(kGaussianExtend, sqrtf(2.0f * logf(op / kAlphaThreshold)));
    }
    if (valid) {
      const float rx = ceilf(extend * sqrtf(cov2d[0]));
      const float ry = ceilf(extend * sqrtf(cov2d[3]));
      valid = !(rx <= p.radius_clip && ry <= p.radius_clip) &&
              !(m2[0] + rx <= 0.0f || m2[0] - rx >= static_cast<float>(p.image_width) || m2[1] + ry <= 0.0f ||
                m2[1] - ry >= static_cast<float>(p.image_height));
      if (valid) {
        const float inv_det = 1.0f / det;
        rx_out = static_cast<int32_t>(rx);
        ry_out = static_cast<int32_t>(ry);
        m2x = m2[0];
        m2y = m2[1];
        depth = mc[2];
        c0 = cov2d[3] * inv_det;
        c1 = -cov2d[1] * inv_det;
        c2 = cov2d[0] * inv_det;
        comp_out = comp;
      }
    }
  }
  radii[idx * 2] = rx_out;
  radii[idx * 2 + 1] = ry_out;
  means2d[idx * 2] = m2x;
  means2d[idx * 2 + 1] = m2y;
  depths[idx] = depth;
  conics[idx * 3] = c0;
  conics[idx * 3 + 1] = c1;
  conics[idx * 3 + 2] = c2;
  if (compensations) compensations[idx] = comp_out;
}

// Opacities of an activated projection without cameras.
__global__ void __launch_bounds__(kProjBlock) sigmoid_kernel(const float* __restrict__ x, int64_t n,
                                                             float* __restrict__ y) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kProjBlock + threadIdx.x;
  if (i < n) y[i] = sigmoid_of(x[i]);
}

// One block per camera: sums the per-block partials and writes the 4x4
// gradient (row 3 zero, column 3 = v_t).
__global__ void __launch_bounds__(256) viewmat_reduce_kernel(const float* __restrict__ partials, int nblk,
                                                             float* __restrict__ v_viewmats) {
  const int64_t cam = blockIdx.x;
  __shared__ float red[256 / kWave][12];
  float acc[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) acc[i] = 0.0f;
  for (int k = threadIdx.x; k < nblk; k += blockDim.x)
#pragma unroll
    for (int i = 0; i < 12; ++i) acc[i] += partials[(cam * nblk + k) * 12 + i];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int i = 0; i < 12; ++i) {
    const float s = wave_sum_uniform(acc[i]);
    if (lane == 0) red[wave][i] = s;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int row = threadIdx.x / 4, col = threadIdx.x % 4;
    float v = 0.0f;
    if (row < 3) {
      const int slot = col < 3 ? row * 3 + col : 9 + row;
#pragma unroll
      for (int w = 0; w < 256 / kWave; ++w) v += red[w][slot];
    }
    v_viewmats[cam * 16 + threadIdx.x] = v;
  }
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

namespace {

// Shared by the operator entry points and the activated ones. `what` names
// the operator in error messages; for ACT the quats / scales / opacities
// arguments carry the raw parameters.
template <bool ACT>
int projection_fwd_impl(const char* what, const float* means, const float* covars, const float* quats,
                        const float* scales, const float* opacities, const float* viewmats, const float* Ks,
                        int64_t B, int64_t C, int64_t N, const gsplat_projection_params* params, int32_t* radii,
                        float* means2d, float* depths, float* conics, float* compensations, float* opac_out,
                        void* stream) {
  const std::string op(what);
  if (!params) return invalid(op + ": null params.");
  if (B < 0 || C < 0 || N < 0) return invalid(op + ": negative size.");
  const gsplat_projection_params& p = *params;
  if (ACT && p.use_covars) return invalid(op + ": the activated projection takes quats and log-scales, not covars.");
  hipStream_t s = as_stream(stream);
  if (B * C * N == 0) {
    // the opacities depend on the Gaussians only (C == 0 still has them)
    if (ACT && opac_out && B * N > 0) {
      if (!opacities) return invalid(op + ": opacities requested without opacity logits.");
      KernelTimer timer("projection_fwd", s);
      sigmoid_kernel<<<grid_for(B * N, kProjBlock), kProjBlock, 0, s>>>(opacities, B * N, opac_out);
      return check_launch(what);
    }
    return GSPLAT_OK;
  }
  if (!means || !viewmats || !Ks || !radii || !means2d || !depths || !conics) return invalid(op + ": null pointer.");
  if (p.use_covars ? !covars : (!quats || !scales)) return invalid(op + " expects covars or quats+scales.");
  if (p.use_opacities && !opacities) return invalid(op + ": null opacities.");
  if (ACT && opac_out && !opacities) return invalid(op + ": opacities requested without opacity logits.");
  if (p.calc_compensations && !compensations) return invalid(op + ": null compensations.");
  if (B * C > 65535) return invalid(op + ": B*C exceeds 65535 cameras.");
  const dim3 grid(grid_for(N, kProjBlock), static_cast<unsigned>(B * C));
  {
    KernelTimer timer("projection_fwd", s);
    projection_fwd_kernel<ACT><<<grid, kProjBlock, 0, s>>>(means, covars, quats, scales, opacities, viewmats, Ks, C,
                                                           N, p, radii, means2d, depths, conics,
                                                           p.calc_compensations ? compensations : nullptr,
                                                           ACT ? opac_out : nullptr);
  }
  return check_launch(what);
}

template <bool ACT>
int projection_bwd_impl(const char* what, const float* means, const float* covars, const float* quats,
                        const float* scales, const float* viewmats, const float* Ks, int64_t B, int64_t C, int64_t N,
                        const gsplat_projection_params* params, const int32_t* radii, const float* conics,
                        const float* compensations, const float* v_means2d, const float* v_depths,
                        const float* v_conics, const float* v_compensations, float* v_means, float* v_covars,
                        float* v_quats, float* v_scales, float* v_viewmats, const float* logits,
                        const float* v_opac, float* v_logits, void* workspace, size_t workspace_bytes,
                        void* stream) {
  const std::string op(what);
  if (!params) return invalid(op + ": null params.");
  const gsplat_projection_params& p = *params;
  if (p.camera_model != 0) return invalid(op + " currently supports pinhole only.");
  if (B < 0 || C < 0 || N < 0) return invalid(op + ": negative size.");
  if (ACT && p.use_covars) return invalid(op + ": the activated projection takes quats and log-scales, not covars.");
  if (ACT && v_logits && !logits) return invalid(op + ": v_opacity_logits requested without opacity logits.");
  hipStream_t s = as_stream(stream);
  if (B * N == 0) {
    if (v_viewmats && B * C > 0) return fill_zero(v_viewmats, B * C * 16 * sizeof(float), s);
    return GSPLAT_OK;
  }
  if (!means || !viewmats || !Ks || !radii || !conics || !v_means2d || !v_conics || !v_means)
    return invalid(op + ": null pointer.");
  if (p.use_covars ? (!covars || !v_covars) : (!quats || !scales || !v_quats || !v_scales))
    return invalid(op + " expects covars or quats+scales.");
  if (v_compensations && !compensations) return invalid(op + ": v_compensations without compensations.");
  if (B > 65535) return invalid(op + ": batch exceeds 65535.");
  float* partials = nullptr;
  if (v_viewmats && C > 0) {
    const size_t need = gsplat_hip_projection_bwd_workspace_size(B, C, N, 1);
    if (!workspace || workspace_bytes < need) {
      set_error(op + ": workspace too small for v_viewmats.");
      return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
    }
    partials = static_cast<float*>(workspace);
  }
  const dim3 grid(grid_for(N, kProjBlock), static_cast<unsigned>(B));
  {
    KernelTimer timer("projection_bwd", s);
    launch_projection_bwd(ACT, grid, s, means, covars, quats, scales, viewmats, Ks, C, N, p, radii, conics,
                          compensations, v_means2d, v_depths, v_conics, v_compensations, v_means, v_covars, v_quats,
                          v_scales, partials, ACT ? logits : nullptr, ACT ? v_opac : nullptr,
                          ACT ? v_logits : nullptr);
  }
  int rc = check_launch(what);
  if (rc != GSPLAT_OK || !v_viewmats) return rc;
  if (C == 0) return GSPLAT_OK;
  {
    KernelTimer timer("projection_bwd_viewmats", s);
    viewmat_reduce_kernel<<<static_cast<unsigned>(B * C), 256, 0, s>>>(partials, static_cast<int>(grid.x), v_viewmats);
  }
  return check_launch(what);
}

}  // namespace

extern "C" int gsplat_hip_projection_fwd(const float* means, const float* covars, const float* quats,
                                         const float* scales, const float* opacities, const float* viewmats,
                                         const float* Ks, int64_t B, int64_t C, int64_t N,
                                         const gsplat_projection_params* params, int32_t* radii, float* means2d,
                                         float* depths, float* conics, float* compensations, void* stream) {
  return projection_fwd_impl<false>("projection_ewa_3dgs_fused_forward", means, covars, quats, scales, opacities,
                                    viewmats, Ks, B, C, N, params, radii, means2d, depths, conics, compensations,
                                    nullptr, stream);
}

extern "C" size_t gsplat_hip_projection_bwd_workspace_size(int64_t B, int64_t C, int64_t N, int32_t viewmats_grad) {
  if (!viewmats_grad || B <= 0 || C <= 0 || N <= 0) return 0;
  return static_cast<size_t>(B * C) * grid_for(N, kProjBlock) * 12 * sizeof(float);
}

extern "C" int gsplat_hip_projection_bwd(const float* means, const float* covars, const float* quats,
                                         const float* scales, const float* viewmats, const float* Ks, int64_t B,
                                         int64_t C, int64_t N, const gsplat_projection_params* params,
                                         const int32_t* radii, const float* conics, const float* compensations,
                                         const float* v_means2d, const float* v_depths, const float* v_conics,
                                         const float* v_compensations, float* v_means, float* v_covars,
                                         float* v_quats, float* v_scales, float* v_viewmats, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  return projection_bwd_impl<false>("projection_ewa_3dgs_fused_backward", means, covars, quats, scales, viewmats, Ks,
                                    B, C, N, params, radii, conics, compensations, v_means2d, v_depths, v_conics,
                                    v_compensations, v_means, v_covars, v_quats, v_scales, v_viewmats, nullptr,
                                    nullptr, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_activated_projection_fwd(const float* means, const float* quats, const float* log_scales,
                                                   const float* opacity_logits, const float* viewmats,
                                                   const float* Ks, int64_t B, int64_t C, int64_t N,
                                                   const gsplat_projection_params* params, int32_t* radii,
                                                   float* means2d, float* depths, float* conics,
                                                   float* compensations, float* opacities, void* stream) {
  return projection_fwd_impl<true>("activated_projection_forward", means, nullptr, quats, log_scales,
                                   opacity_logits, viewmats, Ks, B, C, N, params, radii, means2d, depths, conics,
                                   compensations, opacities, stream);
}

extern "C" int gsplat_hip_activated_projection_bwd(
    const float* means, const float* quats, const float* log_scales, const float* opacity_logits,
    const float* viewmats, const float* Ks, int64_t B, int64_t C, int64_t N, const gsplat_projection_params* params,
    const int32_t* radii, const float* conics, const float* compensations, const float* v_means2d,
    const float* v_depths, const float* v_conics, const float* v_compensations, const float* v_opacities,
    float* v_means, float* v_quats, float* v_log_scales, float* v_opacity_logits, float* v_viewmats,
    void* workspace, size_t workspace_bytes, void* stream) {
  return projection_bwd_impl<true>("activated_projection_backward", means, nullptr, quats, log_scales, viewmats, Ks,
                                   B, C, N, params, radii, conics, compensations, v_means2d, v_depths, v_conics,
                                   v_compensations, v_means, nullptr, v_quats, v_log_scales, v_viewmats,
                                   opacity_logits, v_opacities, v_opacity_logits, workspace, workspace_bytes,
                                   stream);
}
