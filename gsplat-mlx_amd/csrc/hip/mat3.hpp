// Small row-major 3x3 helpers used by the covariance and projection kernels.
// Loop orders (and so float32 rounding) follow the reference CPU helpers in
// gsplat_core/gsplat_quat_scale_to_covar.cpp:103-164 and
// gsplat_core/gsplat_projection.cpp:162-260.
#pragma once

#include <hip/hip_runtime.h>

namespace gsplat_hip {

struct Mat3 {
  float v[9];
};

__device__ __forceinline__ Mat3 mat3_mul(const Mat3& a, const Mat3& b) {
  Mat3 o;
#pragma unroll
  for (int r = 0; r < 3; ++r)
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 3; ++k) acc += a.v[r * 3 + k] * b.v[k * 3 + c];
      o.v[r * 3 + c] = acc;
    }
  return o;
}

__device__ __forceinline__ Mat3 mat3_tr(const Mat3& a) {
  Mat3 o;
  o.v[0] = a.v[0]; o.v[1] = a.v[3]; o.v[2] = a.v[6];
  o.v[3] = a.v[1]; o.v[4] = a.v[4]; o.v[5] = a.v[7];
  o.v[6] = a.v[2]; o.v[7] = a.v[5]; o.v[8] = a.v[8];
  return o;
}

// wxyz quaternion -> rotation (normalised by division).
__device__ __forceinline__ Mat3 quat_to_rotmat(const float q[4]) {
  float w = q[0], x = q[1], y = q[2], z = q[3];
  const float norm = sqrtf(w * w + x * x + y * y + z * z);
  w /= norm;
  x /= norm;
  y /= norm;
  z /= norm;
  const float x2 = x * x, y2 = y * y, z2 = z * z;
  const float xy = x * y, xz = x * z, yz = y * z;
  const float wx = w * x, wy = w * y, wz = w * z;
  Mat3 r;
  r.v[0] = 1.0f - 2.0f * (y2 + z2);
  r.v[1] = 2.0f * (xy - wz);
  r.v[2] = 2.0f * (xz + wy);
  r.v[3] = 2.0f * (xy + wz);
  r.v[4] = 1.0f - 2.0f * (x2 + z2);
  r.v[5] = 2.0f * (yz - wx);
  r.v[6] = 2.0f * (xz - wy);
  r.v[7] = 2.0f * (yz + wx);
  r.v[8] = 1.0f - 2.0f * (x2 + y2);
  return r;
}

// R diag(s^2) R^T, or R diag(s^-2) R^T when `precision`.
__device__ __forceinline__ Mat3 rot_scale_matrix(const Mat3& r, const float scale[3], bool precision) {
  float s[3] = {scale[0], scale[1], scale[2]};
  if (precision) {
    s[0] = 1.0f / s[0];
    s[1] = 1.0f / s[1];
    s[2] = 1.0f / s[2];
  }
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

}  // namespace gsplat_hip
