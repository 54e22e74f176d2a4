// The elementwise glue a training step wraps around the operator chain,
// fused into one kernel per direction instead of a dozen framework launches:
//
//   parameter activations (scanner_points_training_utils.py:39-41, 306-316):
//     quats_n = quats / max(|quats|, 1e-8), scales = exp(log_scales),
//     opacities = sigmoid(opacity_logits) = 1 / (1 + exp(-x));
//   the image L1 term (mean |render - target|).
//
// Forward values use the same operations as the framework composition
// (sum of squares in index order, sqrt, max, divide; expf; 1 / (1 + expf(-x))),
// so they agree to the last bit or two. Gradients:
//   v_quats      = (v_n - n (v_n . n)) / |q|   when |q| >= 1e-8, else v_n / 1e-8
//   v_log_scales = v_scales * scales
//   v_logits     = v_opacities * (1 - o) * o
//   v_render     = (g / count) * sign(render - target), v_target = -v_render.
#include <algorithm>

#include "common.hpp"

namespace gsplat_hip {
namespace {

constexpr int kGlueBlock = 256;

__global__ void __launch_bounds__(kGlueBlock) activations_fwd_kernel(const float* __restrict__ quats,
                                                                     const float* __restrict__ log_scales,
                                                                     const float* __restrict__ logits, int64_t n,
                                                                     float* __restrict__ quats_out,
                                                                     float* __restrict__ scales_out,
                                                                     float* __restrict__ opac_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kGlueBlock + threadIdx.x;
  if (i >= n) return;
  if (quats) {
    const float q0 = quats[i * 4], q1 = quats[i * 4 + 1], q2 = quats[i * 4 + 2], q3 = quats[i * 4 + 3];
    const float ss = ((q0 * q0 + q1 * q1) + q2 * q2) + q3 * q3;
    const float r = sqrtf(ss);
    const float norm = r < 1.0e-8f ? 1.0e-8f : r;  // clamp(min=1e-8); NaN stays NaN
    quats_out[i * 4] = q0 / norm;
    quats_out[i * 4 + 1] = q1 / norm;
    quats_out[i * 4 + 2] = q2 / norm;
    quats_out[i * 4 + 3] = q3 / norm;
  }
  if (log_scales) {
#pragma unroll
    for (int k = 0; k < 3; ++k) scales_out[i * 3 + k] = expf(log_scales[i * 3 + k]);
  }
  if (logits) opac_out[i] = 1.0f / (1.0f + expf(-logits[i]));
}

__global__ void __launch_bounds__(kGlueBlock) activations_bwd_kernel(
    const float* __restrict__ quats, const float* __restrict__ scales, const float* __restrict__ opac,
    const float* __restrict__ v_quats_out, const float* __restrict__ v_scales, const float* __restrict__ v_opac,
    int64_t n, float* __restrict__ v_quats, float* __restrict__ v_log_scales, float* __restrict__ v_logits) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kGlueBlock + threadIdx.x;
  if (i >= n) return;
  if (v_quats) {
    float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (v_quats_out) {
      const float q[4] = {quats[i * 4], quats[i * 4 + 1], quats[i * 4 + 2], quats[i * 4 + 3]};
      const float v[4] = {v_quats_out[i * 4], v_quats_out[i * 4 + 1], v_quats_out[i * 4 + 2], v_quats_out[i * 4 + 3]};
      const float norm = sqrtf(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
      if (norm >= 1.0e-8f) {
        float nq[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) nq[k] = q[k] / norm;
        const float dot = ((v[0] * nq[0] + v[1] * nq[1]) + v[2] * nq[2]) + v[3] * nq[3];
#pragma unroll
        for (int k = 0; k < 4; ++k) g[k] = (v[k] - nq[k] * dot) / norm;
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) g[k] = v[k] / 1.0e-8f;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) v_quats[i * 4 + k] = g[k];
  }
  if (v_log_scales) {
#pragma unroll
    for (int k = 0; k < 3; ++k) v_log_scales[i * 3 + k] = v_scales ? v_scales[i * 3 + k] * scales[i * 3 + k] : 0.0f;
  }
  if (v_logits) {
    const float o = opac[i];
    v_logits[i] = v_opac ? (v_opac[i] * (1.0f - o)) * o : 0.0f;
  }
}

// L1: block partial sums of |a - b| (16-byte loads when aligned), then one
// block adds the partials in a fixed order and divides by the count.
constexpr int kL1Blocks = 1024;

__global__ void __launch_bounds__(kGlueBlock) l1_partial_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ b, int64_t n,
                                                                float* __restrict__ partial) {
  __shared__ float s_w[kGlueBlock / kWave];
  const int t = threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGlueBlock;
  float acc = 0.0f;
  if ((reinterpret_cast<uintptr_t>(a) & 15) == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0) {
    const float4* a4 = reinterpret_cast<const float4*>(a);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    const int64_t n4 = n / 4;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kGlueBlock + t; i < n4; i += stride) {
      const float4 x = a4[i], y = b4[i];
      acc += (fabsf(x.x - y.x) + fabsf(x.y - y.y)) + (fabsf(x.z - y.z) + fabsf(x.w - y.w));
    }
    for (int64_t i = 4 * n4 + static_cast<int64_t>(blockIdx.x) * kGlueBlock + t; i < n; i += stride)
      acc += fabsf(a[i] - b[i]);
  } else {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kGlueBlock + t; i < n; i += stride) acc += fabsf(a[i] - b[i]);
  }
  const float w = wave_sum_uniform(acc);
  if (t % kWave == 0) s_w[t / kWave] = w;
  __syncthreads();
  if (t == 0) {
    float sum = 0.0f;
    for (int k = 0; k < kGlueBlock / kWave; ++k) sum += s_w[k];
    partial[blockIdx.x] = sum;
  }
}

__global__ void __launch_bounds__(kGlueBlock) l1_final_kernel(const float* __restrict__ partial, int parts, int64_t n,
                                                              float* __restrict__ loss) {
  __shared__ float s_w[kGlueBlock / kWave];
  const int t = threadIdx.x;
  constexpr int kPer = kL1Blocks / kGlueBlock;
  float pv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) pv[j] = t + j * kGlueBlock < parts ? partial[t + j * kGlueBlock] : 0.0f;
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) acc += pv[j];
  const float w = wave_sum_uniform(acc);
  if (t % kWave == 0) s_w[t / kWave] = w;
  __syncthreads();
  if (t == 0) {
    float sum = 0.0f;
    for (int k = 0; k < kGlueBlock / kWave; ++k) sum += s_w[k];
    *loss = sum / static_cast<float>(n);
  }
}

__device__ __forceinline__ float sign_of(float x) { return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : (x == x ? 0.0f : x)); }

// One float4 of the operands per thread (16-byte accesses when every
// pointer is aligned; 4-byte ones otherwise).
__global__ void __launch_bounds__(kGlueBlock) l1_bwd_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                            int64_t n, const float* __restrict__ grad,
                                                            float* __restrict__ v_a, float* __restrict__ v_b,
                                                            bool vec) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kGlueBlock + threadIdx.x) * 4;
  if (i0 >= n) return;
  const float g = *grad / static_cast<float>(n);
  if (vec && i0 + 4 <= n) {
    const float4 x = *reinterpret_cast<const float4*>(a + i0);
    const float4 y = *reinterpret_cast<const float4*>(b + i0);
    const float4 v = make_float4(g * sign_of(x.x - y.x), g * sign_of(x.y - y.y), g * sign_of(x.z - y.z),
                                 g * sign_of(x.w - y.w));
    if (v_a) *reinterpret_cast<float4*>(v_a + i0) = v;
    if (v_b) *reinterpret_cast<float4*>(v_b + i0) = make_float4(-v.x, -v.y, -v.z, -v.w);
    return;
  }
  for (int64_t i = i0; i < min<int64_t>(n, i0 + 4); ++i) {
    const float v = g * sign_of(a[i] - b[i]);
    if (v_a) v_a[i] = v;
    if (v_b) v_b[i] = -v;
  }
}

// Selective Adam (upstream gsplat's fused selective_adam_update,
// note/gsplat_cuda_source_map.md:575-577): one lane per value; rows whose
// valid flag is 0 keep their parameter and moments. Adam in torch's form:
// m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g^2,
// p -= (lr / bc1) m / (sqrt(v) / bc2_sqrt + eps); bc1 = bc2_sqrt = 1 gives
// upstream's uncorrected update. The host forms 1 - b1, 1 - b2 and lr / bc1
// in double, as torch does from its Python-float hyperparameters.
__global__ void __launch_bounds__(kGlueBlock) selective_adam_kernel(float* __restrict__ param,
                                                                    const float* __restrict__ grad,
                                                                    float* __restrict__ exp_avg,
                                                                    float* __restrict__ exp_avg_sq,
                                                                    const uint8_t* __restrict__ valid, int64_t n,
                                                                    int64_t D, float step_size, float b1,
                                                                    float omb1, float b2, float omb2, float eps,
                                                                    float bc2_sqrt) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kGlueBlock + threadIdx.x;
  if (i >= n * D) return;
  if (valid && !valid[i / D]) return;
  const float g = grad[i];
  const float m = b1 * exp_avg[i] + omb1 * g;
  const float v = b2 * exp_avg_sq[i] + omb2 * (g * g);
  exp_avg[i] = m;
  exp_avg_sq[i] = v;
  param[i] = param[i] - step_size * (m / (sqrtf(v) / bc2_sqrt + eps));
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" int gsplat_hip_gaussian_activations_fwd(const float* quats, const float* log_scales,
                                                   const float* opacity_logits, int64_t n, float* quats_out,
                                                   float* scales_out, float* opacities_out, void* stream) {
  if (n < 0) return invalid("gaussian_activations_forward: negative size.");
  if (n == 0) return GSPLAT_OK;
  if ((quats && !quats_out) || (log_scales && !scales_out) || (opacity_logits && !opacities_out))
    return invalid("gaussian_activations_forward: null output.");
  if (n > kMaxGridX / 2 * kGlueBlock) return invalid("gaussian_activations_forward: too many Gaussians.");
  hipStream_t s = as_stream(stream);
  {
    KernelTimer timer("activations_fwd", s);
    activations_fwd_kernel<<<grid_for(n, kGlueBlock), kGlueBlock, 0, s>>>(quats, log_scales, opacity_logits, n,
                                                                          quats_out, scales_out, opacities_out);
  }
  return check_launch("gaussian_activations_forward");
}

extern "C" int gsplat_hip_gaussian_activations_bwd(const float* quats, const float* scales, const float* opacities,
                                                   const float* v_quats_out, const float* v_scales,
                                                   const float* v_opacities, int64_t n, float* v_quats,
                                                   float* v_log_scales, float* v_logits, void* stream) {
  if (n < 0) return invalid("gaussian_activations_backward: negative size.");
  if (n == 0) return GSPLAT_OK;
  if ((v_quats && v_quats_out && !quats) || (v_log_scales && v_scales && !scales) || (v_logits && !opacities))
    return invalid("gaussian_activations_backward: null input.");
  if (n > kMaxGridX / 2 * kGlueBlock) return invalid("gaussian_activations_backward: too many Gaussians.");
  hipStream_t s = as_stream(stream);
  {
    KernelTimer timer("activations_bwd", s);
    activations_bwd_kernel<<<grid_for(n, kGlueBlock), kGlueBlock, 0, s>>>(
        quats, scales, opacities, v_quats_out, v_scales, v_opacities, n, v_quats, v_log_scales, v_logits);
  }
  return check_launch("gaussian_activations_backward");
}

extern "C" size_t gsplat_hip_l1_loss_workspace_size(int64_t n) {
  return n > 0 ? static_cast<size_t>(kL1Blocks) * sizeof(float) : 0;
}

extern "C" int gsplat_hip_l1_loss_fwd(const float* a, const float* b, int64_t n, float* loss, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (n < 0) return invalid("l1_loss_forward: negative size.");
  if (!loss) return invalid("l1_loss_forward: null output.");
  hipStream_t s = as_stream(stream);
  if (n == 0) {
    // mean of nothing: 0 / 0 = NaN, as the framework's mean
    l1_final_kernel<<<1, kGlueBlock, 0, s>>>(nullptr, 0, 0, loss);
    return check_launch("l1_loss_forward");
  }
  if (!a || !b) return invalid("l1_loss_forward: null input.");
  if (!workspace || workspace_bytes < gsplat_hip_l1_loss_workspace_size(n)) {
    set_error("l1_loss_forward: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  float* partial = static_cast<float*>(workspace);
  const int parts = static_cast<int>(std::min<int64_t>(kL1Blocks, (n + 4 * kGlueBlock - 1) / (4 * kGlueBlock)));
  {
    KernelTimer timer("l1_loss_fwd", s);
    l1_partial_kernel<<<parts, kGlueBlock, 0, s>>>(a, b, n, partial);
    l1_final_kernel<<<1, kGlueBlock, 0, s>>>(partial, parts, n, loss);
  }
  return check_launch("l1_loss_forward");
}

extern "C" int gsplat_hip_l1_loss_bwd(const float* a, const float* b, int64_t n, const float* grad, float* v_a,
                                      float* v_b, void* stream) {
  if (n < 0) return invalid("l1_loss_backward: negative size.");
  if (n == 0) return GSPLAT_OK;
  if (!a || !b || !grad) return invalid("l1_loss_backward: null input.");
  if ((n + 3) / 4 > static_cast<int64_t>(kMaxGridX / 2) * kGlueBlock)
    return invalid("l1_loss_backward: too many values.");
  hipStream_t s = as_stream(stream);
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = aligned(a) && aligned(b) && (!v_a || aligned(v_a)) && (!v_b || aligned(v_b));
  {
    KernelTimer timer("l1_loss_bwd", s);
    l1_bwd_kernel<<<grid_for((n + 3) / 4, kGlueBlock), kGlueBlock, 0, s>>>(a, b, n, grad, v_a, v_b, vec);
  }
  return check_launch("l1_loss_backward");
}

extern "C" int gsplat_hip_selective_adam(float* param, const float* grad, float* exp_avg, float* exp_avg_sq,
                                         const uint8_t* valid, int64_t n, int64_t D, double lr, double b1, double b2,
                                         double eps, double bias_correction1, double bias_correction2_sqrt,
                                         void* stream) {
  if (n < 0 || D < 0) return invalid("selective_adam: negative size.");
  if (n * D == 0) return GSPLAT_OK;
  if (!param || !grad || !exp_avg || !exp_avg_sq) return invalid("selective_adam: null pointer.");
  if (!(bias_correction1 > 0.0) || !(bias_correction2_sqrt > 0.0))
    return invalid("selective_adam: bias corrections must be positive.");
  hipStream_t s = as_stream(stream);
  {
    KernelTimer timer("selective_adam", s);
    selective_adam_kernel<<<grid_for(n * D, kGlueBlock), kGlueBlock, 0, s>>>(
        param, grad, exp_avg, exp_avg_sq, valid, n, D, static_cast<float>(lr / bias_correction1),
        static_cast<float>(b1), static_cast<float>(1.0 - b1), static_cast<float>(b2), static_cast<float>(1.0 - b2),
        static_cast<float>(eps), static_cast<float>(bias_correction2_sqrt));
  }
  return check_launch("selective_adam");
}
