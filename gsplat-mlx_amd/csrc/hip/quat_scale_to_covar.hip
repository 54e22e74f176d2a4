// quat_scale_to_covar_preci forward / backward for gfx950.
//
// One Gaussian per lane. Arithmetic follows the reference CPU loops
// (gsplat_core/gsplat_quat_scale_to_covar.cpp:103-333) operation for
// operation; this file is compiled with FMA contraction off so float32
// results round like the reference's.
#include "common.hpp"
#include "mat3.hpp"

namespace gsplat_hip {
namespace {

__device__ __forceinline__ void write_matrix(const Mat3& m, bool triu, float* __restrict__ out) {
  if (triu) {
    out[0] = m.v[0];
    out[1] = m.v[1];
    out[2] = m.v[2];
    out[3] = m.v[4];
    out[4] = m.v[5];
    out[5] = m.v[8];
  } else {
#pragma unroll
    for (int i = 0; i < 9; ++i) out[i] = m.v[i];
  }
}

// gsplat_quat_scale_to_covar.cpp:215-236
__device__ __forceinline__ Mat3 cotangent_matrix(bool triu, const float* __restrict__ c) {
  Mat3 o;
  if (triu) {
    o.v[0] = c[0];
    o.v[1] = 0.5f * c[1];
    o.v[2] = 0.5f * c[2];
    o.v[3] = 0.5f * c[1];
    o.v[4] = c[3];
    o.v[5] = 0.5f * c[4];
    o.v[6] = 0.5f * c[2];
    o.v[7] = 0.5f * c[4];
    o.v[8] = c[5];
  } else {
#pragma unroll
    for (int i = 0; i < 9; ++i) o.v[i] = c[i];
  }
  return o;
}

// gsplat_quat_scale_to_covar.cpp:238-276
__device__ __forceinline__ void quat_to_rotmat_vjp_qs(const float q[4], const Mat3& g, float vq[4]) {
  float w = q[0], x = q[1], y = q[2], z = q[3];
  const float norm = sqrtf(w * w + x * x + y * y + z * z);
  const float inv_norm = 1.0f / norm;
  w *= inv_norm;
  x *= inv_norm;
  y *= inv_norm;
  z *= inv_norm;
  const float* r = g.v;
  const float n1 = 2.0f * y * r[1] + 2.0f * z * r[2] + 2.0f * y * r[3] - 4.0f * x * r[4] -
                   2.0f * w * r[5] + 2.0f * z * r[6] + 2.0f * w * r[7] - 4.0f * x * r[8];
  const float n2 = -4.0f * y * r[0] + 2.0f * x * r[1] + 2.0f * w * r[2] + 2.0f * x * r[3] +
                   2.0f * z * r[5] - 2.0f * w * r[6] + 2.0f * z * r[7] - 4.0f * y * r[8];
  const float n3 = -4.0f * z * r[0] - 2.0f * w * r[1] + 2.0f * x * r[2] + 2.0f * w * r[3] -
                   4.0f * z * r[4] + 2.0f * y * r[5] + 2.0f * x * r[6] + 2.0f * y * r[7];
  const float n0 = -2.0f * z * r[1] + 2.0f * y * r[2] + 2.0f * z * r[3] - 2.0f * x * r[5] -
                   2.0f * y * r[6] + 2.0f * x * r[7];
  const float dot = n0 * w + n1 * x + n2 * y + n3 * z;
  vq[0] += (n0 - dot * w) * inv_norm;
  vq[1] += (n1 - dot * x) * inv_norm;
  vq[2] += (n2 - dot * y) * inv_norm;
  vq[3] += (n3 - dot * z) * inv_norm;
}

// gsplat_quat_scale_to_covar.cpp:278-333
__device__ __forceinline__ void quat_scale_vjp(const float q[4], const float sc[3], const Mat3& r,
                                               const Mat3& vm, bool precision, float vq[4],
                                               float vs[3]) {
  float s[3] = {sc[0], sc[1], sc[2]};
  if (precision) {
    s[0] = 1.0f / s[0];
    s[1] = 1.0f / s[1];
    s[2] = 1.0f / s[2];
  }
  Mat3 m, v_m, v_r;
#pragma unroll
  for (int row = 0; row < 3; ++row)
#pragma unroll
    for (int col = 0; col < 3; ++col) m.v[row * 3 + col] = r.v[row * 3 + col] * s[col];
#pragma unroll
  for (int row = 0; row < 3; ++row)
#pragma unroll
    for (int col = 0; col < 3; ++col) {
      float value = 0.0f;
#pragma unroll
      for (int k = 0; k < 3; ++k) value += (vm.v[row * 3 + k] + vm.v[k * 3 + row]) * m.v[k * 3 + col];
      v_m.v[row * 3 + col] = value;
    }
#pragma unroll
  for (int row = 0; row < 3; ++row)
#pragma unroll
    for (int col = 0; col < 3; ++col) v_r.v[row * 3 + col] = v_m.v[row * 3 + col] * s[col];
  quat_to_rotmat_vjp_qs(q, v_r, vq);
#pragma unroll
  for (int col = 0; col < 3; ++col) {
    float grad = 0.0f;
#pragma unroll
    for (int row = 0; row < 3; ++row) grad += r.v[row * 3 + col] * v_m.v[row * 3 + col];
    if (precision)
      vs[col] += -s[col] * s[col] * grad;
    else
      vs[col] += grad;
  }
}

__global__ void __launch_bounds__(256) qs_fwd_kernel(const float* __restrict__ quats,
                                                     const float* __restrict__ scales, int64_t n,
                                                     int compute_covar, int compute_preci, int triu,
                                                     float* __restrict__ covars,
                                                     float* __restrict__ precis) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const float q[4] = {quats[e * 4], quats[e * 4 + 1], quats[e * 4 + 2], quats[e * 4 + 3]};
  const float s[3] = {scales[e * 3], scales[e * 3 + 1], scales[e * 3 + 2]};
  const Mat3 r = quat_to_rotmat(q);
  const int stride = triu ? 6 : 9;
  if (compute_covar) write_matrix(rot_scale_matrix(r, s, false), triu != 0, covars + e * stride);
  if (compute_preci) write_matrix(rot_scale_matrix(r, s, true), triu != 0, precis + e * stride);
}

__global__ void __launch_bounds__(256) qs_bwd_kernel(const float* __restrict__ quats,
                                                     const float* __restrict__ scales,
                                                     const float* __restrict__ v_covars,
                                                     const float* __restrict__ v_precis, int64_t n,
                                                     int triu, float* __restrict__ v_quats,
                                                     float* __restrict__ v_scales) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const float q[4] = {quats[e * 4], quats[e * 4 + 1], quats[e * 4 + 2], quats[e * 4 + 3]};
  const float s[3] = {scales[e * 3], scales[e * 3 + 1], scales[e * 3 + 2]};
  const int stride = triu ? 6 : 9;
  float vq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float vs[3] = {0.0f, 0.0f, 0.0f};
  const Mat3 r = quat_to_rotmat(q);
  if (v_covars) quat_scale_vjp(q, s, r, cotangent_matrix(triu != 0, v_covars + e * stride), false, vq, vs);
  if (v_precis) quat_scale_vjp(q, s, r, cotangent_matrix(triu != 0, v_precis + e * stride), true, vq, vs);
#pragma unroll
  for (int i = 0; i < 4; ++i) v_quats[e * 4 + i] = vq[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) v_scales[e * 3 + i] = vs[i];
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" int gsplat_hip_quat_scale_to_covar_preci_fwd(const float* quats, const float* scales, int64_t n,
                                                        int32_t compute_covar, int32_t compute_preci,
                                                        int32_t triu, float* covars, float* precis,
                                                        void* stream) {
  if (n < 0) return invalid("quat_scale_to_covar_preci_forward: negative size.");
  if (n == 0) return GSPLAT_OK;
  if (!quats || !scales || (compute_covar && !covars) || (compute_preci && !precis))
    return invalid("quat_scale_to_covar_preci_forward: null pointer.");
  if (grid_for(n, 256) > kMaxGridX) return invalid("quat_scale_to_covar_preci_forward: too many elements.");
  {
    KernelTimer timer("quat_scale_to_covar_fwd", as_stream(stream));
    qs_fwd_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(quats, scales, n, compute_covar, compute_preci,
                                                                    triu, covars, precis);
  }
  return check_launch("quat_scale_to_covar_preci_forward");
}

extern "C" int gsplat_hip_quat_scale_to_covar_preci_bwd(const float* quats, const float* scales,
                                                        const float* v_covars, const float* v_precis,
                                                        int64_t n, int32_t triu, float* v_quats,
                                                        float* v_scales, void* stream) {
  if (n < 0) return invalid("quat_scale_to_covar_preci_backward: negative size.");
  if (n == 0) return GSPLAT_OK;
  if (!quats || !scales || !v_quats || !v_scales)
    return invalid("quat_scale_to_covar_preci_backward: null pointer.");
  {
    KernelTimer timer("quat_scale_to_covar_bwd", as_stream(stream));
    qs_bwd_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(quats, scales, v_covars, v_precis, n, triu,
                                                                    v_quats, v_scales);
  }
  return check_launch("quat_scale_to_covar_preci_backward");
}
