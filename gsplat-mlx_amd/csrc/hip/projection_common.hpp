// Per-Gaussian helpers shared by the projection forward (projection.hip,
// compiled with FMA contraction off and correctly rounded division: its
// outputs round like the reference's float32 loops) and backward
// (projection_bwd.hip, compiled with FMA contraction and fast division: only
// gradients, held to a relative tolerance). Each translation unit compiles
// its own copy with its own flags.
#pragma once

#include "common.hpp"
#include "mat3.hpp"

namespace gsplat_hip {

// Launches the projection backward kernel (projection_bwd.hip); arguments as
// gsplat_hip_projection_bwd, plus the activated projection's opacity logits,
// opacities' cotangent and logits' gradient (act). With pmask / pprefix (the
// packed layout's bit per pair and per-word prefix), radii is unused and the
// per-pair arrays are read at the pair's packed row.
void launch_projection_bwd(bool act, dim3 grid, hipStream_t s, const float* means, const float* covars,
                           const float* quats, const float* scales, const float* viewmats, const float* Ks, int64_t C,
                           int64_t N, const gsplat_projection_params& p, const int32_t* radii, const float* conics,
                           const float* compensations, const float* v_means2d, const float* v_depths,
                           const float* v_conics, const float* v_compensations, float* v_means, float* v_covars,
                           float* v_quats, float* v_scales, float* vm_partials, const float* logits,
                           const float* v_opac, float* v_logits, const uint64_t* pmask = nullptr,
                           const int32_t* pprefix = nullptr, const float* v_opac_rows = nullptr,
                           float* v_viewspace = nullptr);

namespace {


constexpr int kProjBlock = 256;

// Parameter activations, the operations of training_glue.hip's kernels.
__device__ __forceinline__ void activate_quat(const float qr[4], float q[4]) {
  const float r = sqrtf(((qr[0] * qr[0] + qr[1] * qr[1]) + qr[2] * qr[2]) + qr[3] * qr[3]);
  const float norm = r < 1.0e-8f ? 1.0e-8f : r;  // clamp(min=1e-8); NaN stays NaN
#pragma unroll
  for (int k = 0; k < 4; ++k) q[k] = qr[k] / norm;
}

// d(quats / max(|quats|, 1e-8)) / d quats applied to v
__device__ __forceinline__ void activate_quat_vjp(const float qr[4], const float v[4], float g[4]) {
  const float norm = sqrtf(((qr[0] * qr[0] + qr[1] * qr[1]) + qr[2] * qr[2]) + qr[3] * qr[3]);
  if (norm >= 1.0e-8f) {
    float nq[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) nq[k] = qr[k] / norm;
    const float dot = ((v[0] * nq[0] + v[1] * nq[1]) + v[2] * nq[2]) + v[3] * nq[3];
#pragma unroll
    for (int k = 0; k < 4; ++k) g[k] = (v[k] - nq[k] * dot) / norm;
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) g[k] = v[k] / 1.0e-8f;
  }
}

__device__ __forceinline__ float sigmoid_of(float x) { return 1.0f / (1.0f + expf(-x)); }

// quaternion and scales of Gaussian g (ACT: activated from the raw parameters)
template <bool ACT>
__device__ __forceinline__ void load_quat_scale(const float* __restrict__ quats, const float* __restrict__ scales,
                                                int64_t g, float q[4], float s[3]) {
  const float qr[4] = {quats[g * 4], quats[g * 4 + 1], quats[g * 4 + 2], quats[g * 4 + 3]};
  if constexpr (ACT) {
    activate_quat(qr, q);
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = expf(scales[g * 3 + k]);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k] = qr[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = scales[g * 3 + k];
  }
}

// The same from values already loaded (raw quaternion qr, scales or
// log-scales sr).
template <bool ACT>
__device__ __forceinline__ void quat_scale_of(const float qr[4], const float sr[3], float q[4], float s[3]) {
  if constexpr (ACT) {
    activate_quat(qr, q);
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = expf(sr[k]);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k] = qr[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = sr[k];
  }
}

struct CamFrame {
  Mat3 R;
  float t[3];
  float fx, fy, cx, cy;
};

__device__ __forceinline__ CamFrame load_camera(const float* __restrict__ view, const float* __restrict__ K) {
  CamFrame f;
  f.R.v[0] = view[0]; f.R.v[1] = view[1]; f.R.v[2] = view[2];
  f.R.v[3] = view[4]; f.R.v[4] = view[5]; f.R.v[5] = view[6];
  f.R.v[6] = view[8]; f.R.v[7] = view[9]; f.R.v[8] = view[10];
  f.t[0] = view[3];
  f.t[1] = view[7];
  f.t[2] = view[11];
  f.fx = K[0];
  f.fy = K[4];
  f.cx = K[2];
  f.cy = K[5];
  return f;
}

__device__ __forceinline__ void world_to_cam(const CamFrame& f, const float mw[3], float mc[3]) {
  const float* R = f.R.v;
  mc[0] = R[0] * mw[0] + R[1] * mw[1] + R[2] * mw[2] + f.t[0];
  mc[1] = R[3] * mw[0] + R[4] * mw[1] + R[5] * mw[2] + f.t[1];
  mc[2] = R[6] * mw[0] + R[7] * mw[1] + R[8] * mw[2] + f.t[2];
}

__device__ __forceinline__ Mat3 read_covar(const float* __restrict__ c) {
  Mat3 m;
  m.v[0] = c[0]; m.v[1] = c[1]; m.v[2] = c[2];
  m.v[3] = c[1]; m.v[4] = c[3]; m.v[5] = c[4];
  m.v[6] = c[2]; m.v[7] = c[4]; m.v[8] = c[5];
  return m;
}

// M M^T with M = R diag(s) (gsplat_projection.cpp:204-218).
__device__ __forceinline__ Mat3 covar_from_quat_scale(const float q[4], const float s[3]) {
  const Mat3 r = quat_to_rotmat(q);
  Mat3 o;
#pragma unroll
  for (int row = 0; row < 3; ++row)
#pragma unroll
    for (int col = 0; col < 3; ++col) {
      float value = 0.0f;
#pragma unroll
      for (int k = 0; k < 3; ++k) value += r.v[row * 3 + k] * s[k] * s[k] * r.v[col * 3 + k];
      o.v[row * 3 + col] = value;
    }
  return o;
}

// Perspective frustum limits (gsplat_projection.cpp:478-488).
struct PerspLimits {
  float lim_x_pos, lim_x_neg, lim_y_pos, lim_y_neg;
};

__device__ __forceinline__ PerspLimits persp_limits(float fx, float fy, float cx, float cy, int width, int height) {
  const float tan_fovx = 0.5f * static_cast<float>(width) / fx;
  const float tan_fovy = 0.5f * static_cast<float>(height) / fy;
  PerspLimits l;
  l.lim_x_pos = (static_cast<float>(width) - cx) / fx + 0.3f * tan_fovx;
  l.lim_x_neg = cx / fx + 0.3f * tan_fovx;
  l.lim_y_pos = (static_cast<float>(height) - cy) / fy + 0.3f * tan_fovy;
  l.lim_y_neg = cy / fy + 0.3f * tan_fovy;
  return l;
}

// J (2x3, row-major) and mean2d for pinhole / orthographic / fisheye
// (gsplat_projection.metal:122-200).
__device__ __forceinline__ void camera_jacobian(int model, const float mc[3], const CamFrame& f, int width,
                                                int height, float J[6], float m2[2]) {
  const float x = mc[0], y = mc[1], z = mc[2];
  if (model == 1) {
    J[0] = f.fx; J[1] = 0.0f; J[2] = 0.0f;
    J[3] = 0.0f; J[4] = f.fy; J[5] = 0.0f;
    m2[0] = f.fx * x + f.cx;
    m2[1] = f.fy * y + f.cy;
    return;
  }
  if (model == 2) {
    const float eps = 0.0000001f;
    const float xy_len = sqrtf(x * x + y * y) + eps;
    const float theta = atan2f(xy_len, z + eps);
    m2[0] = x * f.fx * theta / xy_len + f.cx;
    m2[1] = y * f.fy * theta / xy_len + f.cy;
    const float x2 = x * x + eps;
    const float y2 = y * y;
    const float xy = x * y;
    const float x2y2 = x2 + y2;
    const float x2y2z2_inv = 1.0f / (x2y2 + z * z);
    const float b = atan2f(xy_len, z) / xy_len / x2y2;
    const float a = z * x2y2z2_inv / x2y2;
    J[0] = f.fx * (x2 * a + y2 * b);
    J[1] = f.fx * xy * (a - b);
    J[2] = -f.fx * x * x2y2z2_inv;
    J[3] = f.fy * xy * (a - b);
    J[4] = f.fy * (y2 * a + x2 * b);
    J[5] = -f.fy * y * x2y2z2_inv;
    return;
  }
  const PerspLimits l = persp_limits(f.fx, f.fy, f.cx, f.cy, width, height);
  const float rz = 1.0f / z;
  const float rz2 = rz * rz;
  const float tx = z * fminf(l.lim_x_pos, fmaxf(-l.lim_x_neg, x * rz));
  const float ty = z * fminf(l.lim_y_pos, fmaxf(-l.lim_y_neg, y * rz));
  J[0] = f.fx * rz; J[1] = 0.0f; J[2] = -f.fx * tx * rz2;
  J[3] = 0.0f; J[4] = f.fy * rz; J[5] = -f.fy * ty * rz2;
  m2[0] = f.fx * x * rz + f.cx;
  m2[1] = f.fy * y * rz + f.cy;
}

}  // namespace
}  // namespace gsplat_hip
