// Fused EWA projection (forward / backward) for gfx950.
//
// Forward: one lane per (camera, Gaussian); blockIdx.y selects the camera so
// viewmat and K are wave-uniform (scalar loads). Culling follows the
// reference GPU kernel (gsplat_core/metal/gsplat_projection.metal:214-339);
// per-Gaussian math follows gsplat_core/gsplat_projection.cpp:446-521 in the
// same operation order (file compiled without FMA contraction).
//
// Backward: one lane per (batch, Gaussian) looping over the C cameras (no
// atomics), as gsplat_projection.metal:446-569. The view-matrix gradient is a
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
#include "common.hpp"
#include "mat3.hpp"

namespace gsplat_hip {
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

// gsplat_projection.cpp:262-284
__device__ __forceinline__ void add_blur_vjp(float eps2d, const float cb[4], float compensation, float v_comp,
                                             float v_cov[4]) {
  const float det_conic_blur = cb[0] * cb[3] - cb[1] * cb[2];
  const float v_sqr_comp = v_comp * 0.5f / (compensation + 1.0e-6f);
  const float one_minus_sqr_comp = 1.0f - compensation * compensation;
  v_cov[0] += v_sqr_comp * (one_minus_sqr_comp * cb[0] - eps2d * det_conic_blur);
  v_cov[1] += v_sqr_comp * (one_minus_sqr_comp * cb[1]);
  v_cov[2] += v_sqr_comp * (one_minus_sqr_comp * cb[2]);
  v_cov[3] += v_sqr_comp * (one_minus_sqr_comp * cb[3] - eps2d * det_conic_blur);
}

// gsplat_projection.cpp:286-377
__device__ __forceinline__ void persp_proj_vjp(const float mc[3], const Mat3& cov3d, const CamFrame& f, int width,
                                               int height, const float v_cov2d[4], const float v_mean2d[2],
                                               float v_mc[3], Mat3& v_cov3d) {
  const float x = mc[0], y = mc[1], z = mc[2];
  const PerspLimits l = persp_limits(f.fx, f.fy, f.cx, f.cy, width, height);
  const float rz = 1.0f / z;
  const float rz2 = rz * rz;
  const float rz3 = rz2 * rz;
  const float x_rz = x * rz;
  const float y_rz = y * rz;
  const float tx = z * fminf(l.lim_x_pos, fmaxf(-l.lim_x_neg, x_rz));
  const float ty = z * fminf(l.lim_y_pos, fmaxf(-l.lim_y_neg, y_rz));
  const float J[6] = {f.fx * rz, 0.0f, -f.fx * tx * rz2, 0.0f, f.fy * rz, -f.fy * ty * rz2};
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      float acc = 0.0f;
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc += J[r * 3 + a] * v_cov2d[r * 2 + c] * J[c * 3 + b];
      v_cov3d.v[a * 3 + b] = acc;
    }
  v_mc[0] += f.fx * rz * v_mean2d[0];
  v_mc[1] += f.fy * rz * v_mean2d[1];
  v_mc[2] += -(f.fx * x * v_mean2d[0] + f.fy * y * v_mean2d[1]) * rz2;
  float v_J[6];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      float left = 0.0f, right = 0.0f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int b = 0; b < 3; ++b) {
          left += v_cov2d[r * 2 + c] * J[c * 3 + b] * cov3d.v[a * 3 + b];
          right += v_cov2d[c * 2 + r] * J[c * 3 + b] * cov3d.v[b * 3 + a];
        }
      v_J[r * 3 + a] = left + right;
    }
  if (x_rz <= l.lim_x_pos && x_rz >= -l.lim_x_neg)
    v_mc[0] += -f.fx * rz2 * v_J[2];
  else
    v_mc[2] += -f.fx * rz3 * tx * v_J[2];
  if (y_rz <= l.lim_y_pos && y_rz >= -l.lim_y_neg)
    v_mc[1] += -f.fy * rz2 * v_J[5];
  else
    v_mc[2] += -f.fy * rz3 * ty * v_J[5];
  v_mc[2] += -f.fx * rz2 * v_J[0] - f.fy * rz2 * v_J[4] + 2.0f * f.fx * tx * rz3 * v_J[2] +
             2.0f * f.fy * ty * rz3 * v_J[5];
}

// gsplat_projection.cpp:404-437
__device__ __forceinline__ void quat_to_rotmat_vjp(const float q[4], const Mat3& v_R, float vq[4]) {
  float w = q[0], x = q[1], y = q[2], z = q[3];
  const float inv_norm = 1.0f / sqrtf(w * w + x * x + y * y + z * z);
  w *= inv_norm;
  x *= inv_norm;
  y *= inv_norm;
  z *= inv_norm;
  const float* g = v_R.v;
  const float n[4] = {
      2.0f * (x * (g[7] - g[5]) + y * (g[2] - g[6]) + z * (g[3] - g[1])),
      2.0f * (-2.0f * x * (g[4] + g[8]) + y * (g[1] + g[3]) + z * (g[2] + g[6]) + w * (g[7] - g[5])),
      2.0f * (x * (g[1] + g[3]) - 2.0f * y * (g[0] + g[8]) + z * (g[5] + g[7]) + w * (g[2] - g[6])),
      2.0f * (x * (g[2] + g[6]) + y * (g[5] + g[7]) - 2.0f * z * (g[0] + g[4]) + w * (g[3] - g[1])),
  };
  const float qn[4] = {w, x, y, z};
  float dot = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) dot += n[i] * qn[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) vq[i] += (n[i] - dot * qn[i]) * inv_norm;
}

// gsplat_projection.cpp:439-474
__device__ __forceinline__ void quat_scale_to_covar_vjp(const float q[4], const float s[3], const Mat3& v_covar,
                                                        float vq[4], float vs[3]) {
  const Mat3 R = quat_to_rotmat(q);
  Mat3 M, sym;
#pragma unroll
  for (int row = 0; row < 3; ++row)
#pragma unroll
    for (int col = 0; col < 3; ++col) {
      M.v[row * 3 + col] = R.v[row * 3 + col] * s[col];
      sym.v[row * 3 + col] = v_covar.v[row * 3 + col] + v_covar.v[col * 3 + row];
    }
  const Mat3 v_M = mat3_mul(sym, M);
  Mat3 v_R;
#pragma unroll
  for (int row = 0; row < 3; ++row)
#pragma unroll
    for (int col = 0; col < 3; ++col) {
      v_R.v[row * 3 + col] = v_M.v[row * 3 + col] * s[col];
      vs[col] += v_M.v[row * 3 + col] * R.v[row * 3 + col];
    }
  quat_to_rotmat_vjp(q, v_R, vq);
}

// Sum of 12 per-lane values over the block; lane 0 of the block writes them.
template <int BLOCK>
__device__ __forceinline__ void block_sum12_store(float vals[12], float* __restrict__ out) {
  __shared__ float red[BLOCK / kWave][12];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int i = 0; i < 12; ++i) {
    const float s = wave_sum_uniform(vals[i]);
    if (lane == 0) red[wave][i] = s;
  }
  __syncthreads();
  if (threadIdx.x < 12) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < BLOCK / kWave; ++w) acc += red[w][threadIdx.x];
    out[threadIdx.x] = acc;
  }
  __syncthreads();
}

// ACT: quats / scales hold quaternions / log-scales (raw), v_quats / v_scales
// receive their gradients, and v_logits (if non-null) = v_opac * o (1 - o)
// with o = sigmoid(logits) (v_opac null: zeros).
template <bool ACT>
__global__ void __launch_bounds__(kProjBlock) projection_bwd_kernel(
    const float* __restrict__ means, const float* __restrict__ covars, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ viewmats, const float* __restrict__ Ks, int64_t C,
    int64_t N, gsplat_projection_params p, const int32_t* __restrict__ radii, const float* __restrict__ conics,
    const float* __restrict__ compensations, const float* __restrict__ v_means2d,
    const float* __restrict__ v_depths, const float* __restrict__ v_conics,
    const float* __restrict__ v_compensations, float* __restrict__ v_means, float* __restrict__ v_covars,
    float* __restrict__ v_quats, float* __restrict__ v_scales, float* __restrict__ vm_partials,
    const float* __restrict__ logits, const float* __restrict__ v_opac, float* __restrict__ v_logits) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kProjBlock + threadIdx.x;
  const int64_t b = blockIdx.y;
  const bool in_range = n < N;
  const int64_t g = b * N + (in_range ? n : 0);

  float mw[3] = {0.0f, 0.0f, 0.0f};
  float q[4] = {1.0f, 0.0f, 0.0f, 0.0f};
  float s[3] = {1.0f, 1.0f, 1.0f};
  Mat3 cw;
  if (in_range) {
    mw[0] = means[g * 3];
    mw[1] = means[g * 3 + 1];
    mw[2] = means[g * 3 + 2];
    if (p.use_covars) {
      cw = read_covar(covars + g * 6);
    } else {
      load_quat_scale<ACT>(quats, scales, g, q, s);
      cw = covar_from_quat_scale(q, s);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 9; ++i) cw.v[i] = 0.0f;
  }

  float v_mw_total[3] = {0.0f, 0.0f, 0.0f};
  Mat3 v_cw_total;
#pragma unroll
  for (int i = 0; i < 9; ++i) v_cw_total.v[i] = 0.0f;

  for (int64_t c = 0; c < C; ++c) {
    const int64_t cam = b * C + c;
    const int64_t idx = cam * N + n;
    const bool valid = in_range && radii[idx * 2] > 0 && radii[idx * 2 + 1] > 0;
    float vm_part[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) vm_part[i] = 0.0f;
    if (valid) {
      const CamFrame f = load_camera(viewmats + cam * 16, Ks + cam * 9);
      const float cn[3] = {conics[idx * 3], conics[idx * 3 + 1], conics[idx * 3 + 2]};
      const float vc[3] = {v_conics[idx * 3], v_conics[idx * 3 + 1], v_conics[idx * 3 + 2]};
      const float inv[4] = {cn[0], cn[1], cn[1], cn[2]};
      const float vinv[4] = {vc[0], 0.5f * vc[1], 0.5f * vc[1], vc[2]};
      const float tmp[4] = {inv[0] * vinv[0] + inv[1] * vinv[2], inv[0] * vinv[1] + inv[1] * vinv[3],
                            inv[2] * vinv[0] + inv[3] * vinv[2], inv[2] * vinv[1] + inv[3] * vinv[3]};
      float v_cov2d[4] = {-(tmp[0] * inv[0] + tmp[1] * inv[2]), -(tmp[0] * inv[1] + tmp[1] * inv[3]),
                          -(tmp[2] * inv[0] + tmp[3] * inv[2]), -(tmp[2] * inv[1] + tmp[3] * inv[3])};
      if (v_compensations) add_blur_vjp(p.eps2d, inv, compensations[idx], v_compensations[idx], v_cov2d);
      float mc[3];
      world_to_cam(f, mw, mc);
      const Mat3 cc = mat3_mul(mat3_mul(f.R, cw), mat3_tr(f.R));
      float v_mc[3] = {0.0f, 0.0f, v_depths ? v_depths[idx] : 0.0f};
      const float vm2[2] = {v_means2d[idx * 2], v_means2d[idx * 2 + 1]};
      Mat3 v_cc;
      persp_proj_vjp(mc, cc, f, p.image_width, p.image_height, v_cov2d, vm2, v_mc, v_cc);
      const float* R = f.R.v;
#pragma unroll
      for (int i = 0; i < 3; ++i) v_mw_total[i] += R[i] * v_mc[0] + R[3 + i] * v_mc[1] + R[6 + i] * v_mc[2];
      const Mat3 v_cw = mat3_mul(mat3_mul(mat3_tr(f.R), v_cc), f.R);
#pragma unroll
      for (int i = 0; i < 9; ++i) v_cw_total.v[i] += v_cw.v[i];
      if (vm_partials) {
        const Mat3 term1 = mat3_mul(mat3_mul(v_cc, f.R), mat3_tr(cw));
        const Mat3 term2 = mat3_mul(mat3_mul(mat3_tr(v_cc), f.R), cw);
#pragma unroll
        for (int row = 0; row < 3; ++row) {
#pragma unroll
          for (int col = 0; col < 3; ++col)
            vm_part[row * 3 + col] = v_mc[row] * mw[col] + term1.v[row * 3 + col] + term2.v[row * 3 + col];
          vm_part[9 + row] = v_mc[row];
        }
      }
    }
    if (vm_partials) {
      // partials layout: [B*C][gridDim.x][12]
      block_sum12_store<kProjBlock>(vm_part, vm_partials + (cam * gridDim.x + blockIdx.x) * 12);
    }
  }
  if (!in_range) return;
#pragma unroll
  for (int i = 0; i < 3; ++i) v_means[g * 3 + i] = v_mw_total[i];
  if (p.use_covars) {
    const float* v = v_cw_total.v;
    float* o = v_covars + g * 6;
    o[0] = v[0];
    o[1] = v[1] + v[3];
    o[2] = v[2] + v[6];
    o[3] = v[4];
    o[4] = v[5] + v[7];
    o[5] = v[8];
  } else {
    float vq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float vs[3] = {0.0f, 0.0f, 0.0f};
    quat_scale_to_covar_vjp(q, s, v_cw_total, vq, vs);
    if constexpr (ACT) {
      const float qr[4] = {quats[g * 4], quats[g * 4 + 1], quats[g * 4 + 2], quats[g * 4 + 3]};
      float vr[4];
      activate_quat_vjp(qr, vq, vr);
#pragma unroll
      for (int i = 0; i < 4; ++i) vq[i] = vr[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) vs[i] = vs[i] * s[i];  // d exp(x) / dx = exp(x)
      if (v_logits) {
        const float o = sigmoid_of(logits[g]);
        v_logits[g] = v_opac ? (v_opac[g] * (1.0f - o)) * o : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v_quats[g * 4 + i] = vq[i];
#pragma unroll
    for (int i = 0; i < 3; ++i) v_scales[g * 3 + i] = vs[i];
  }
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
    projection_bwd_kernel<ACT><<<grid, kProjBlock, 0, s>>>(
        means, covars, quats, scales, viewmats, Ks, C, N, p, radii, conics, compensations, v_means2d, v_depths,
        v_conics, v_compensations, v_means, v_covars, v_quats, v_scales, partials, ACT ? logits : nullptr,
        ACT ? v_opac : nullptr, ACT ? v_logits : nullptr);
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
