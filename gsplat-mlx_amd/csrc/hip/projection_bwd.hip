// Fused EWA projection backward for gfx950 (the kernel that
// gsplat_hip_projection_bwd and gsplat_hip_activated_projection_bwd launch;
// see projection.hip). Gradient arithmetic only, so this file is compiled
// with FMA contraction and fast float32 division and square root; the
// results stay within the chain's gradient tolerance of the exact ones.
#include "projection_common.hpp"

namespace gsplat_hip {
namespace {

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
// Orthographic camera: J = [[fx, 0, 0], [0, fy, 0]] is constant, so
// v_cov3d = J^T v_cov2d J and v_mc += (fx v_mean2d.x, fy v_mean2d.y, 0)
// (upstream gsplat's ortho_proj_vjp; the reference guards every non-pinhole
// backward, gsplat_projection.cpp:157-160).
__device__ __forceinline__ void ortho_proj_vjp(const CamFrame& f, const float v_cov2d[4], const float v_mean2d[2],
                                               float v_mc[3], Mat3& v_cov3d) {
  const float J[6] = {f.fx, 0.0f, 0.0f, 0.0f, f.fy, 0.0f};
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
  v_mc[0] += f.fx * v_mean2d[0];
  v_mc[1] += f.fy * v_mean2d[1];
}

// Equidistant fisheye (upstream gsplat's fisheye_proj_vjp; the reference has
// the forward only, camera_jacobian): the mean's image point and the EWA
// Jacobian J are nonlinear in the camera-space mean, so their derivatives
// are carried as forward-mode dual numbers through the forward's own
// formulas (value + d/dx, d/dy, d/dz), which differentiates exactly what the
// forward computes, eps terms included.
struct Dual3 {
  float v, d[3];
};
__device__ __forceinline__ Dual3 dconst(float c) { return {c, {0.0f, 0.0f, 0.0f}}; }
__device__ __forceinline__ Dual3 operator+(const Dual3& a, const Dual3& b) {
  return {a.v + b.v, {a.d[0] + b.d[0], a.d[1] + b.d[1], a.d[2] + b.d[2]}};
}
__device__ __forceinline__ Dual3 operator-(const Dual3& a, const Dual3& b) {
  return {a.v - b.v, {a.d[0] - b.d[0], a.d[1] - b.d[1], a.d[2] - b.d[2]}};
}
__device__ __forceinline__ Dual3 operator*(const Dual3& a, const Dual3& b) {
  return {a.v * b.v, {a.d[0] * b.v + a.v * b.d[0], a.d[1] * b.v + a.v * b.d[1], a.d[2] * b.v + a.v * b.d[2]}};
}
__device__ __forceinline__ Dual3 operator/(const Dual3& a, const Dual3& b) {
  const float q = a.v / b.v;
  return {q, {(a.d[0] - q * b.d[0]) / b.v, (a.d[1] - q * b.d[1]) / b.v, (a.d[2] - q * b.d[2]) / b.v}};
}
__device__ __forceinline__ Dual3 dsqrt(const Dual3& a) {
  const float r = sqrtf(a.v);
  const float k = 0.5f / r;
  return {r, {a.d[0] * k, a.d[1] * k, a.d[2] * k}};
}
// atan2(u, w): d = (w du - u dw) / (u^2 + w^2)
__device__ __forceinline__ Dual3 datan2(const Dual3& u, const Dual3& w) {
  const float den = u.v * u.v + w.v * w.v;
  Dual3 o;
  o.v = atan2f(u.v, w.v);
#pragma unroll
  for (int k = 0; k < 3; ++k) o.d[k] = (w.v * u.d[k] - u.v * w.d[k]) / den;
  return o;
}

__device__ __forceinline__ void fisheye_proj_vjp(const float mc[3], const Mat3& cov3d, const CamFrame& f,
                                                 const float v_cov2d[4], const float v_mean2d[2], float v_mc[3],
                                                 Mat3& v_cov3d) {
  const Dual3 x = {mc[0], {1.0f, 0.0f, 0.0f}}, y = {mc[1], {0.0f, 1.0f, 0.0f}}, z = {mc[2], {0.0f, 0.0f, 1.0f}};
  const Dual3 eps = dconst(0.0000001f), fx = dconst(f.fx), fy = dconst(f.fy);
  const Dual3 xy_len = dsqrt(x * x + y * y) + eps;
  const Dual3 theta = datan2(xy_len, z + eps);
  const Dual3 m2x = x * fx * theta / xy_len;
  const Dual3 m2y = y * fy * theta / xy_len;
  const Dual3 x2 = x * x + eps, y2 = y * y, xy = x * y;
  const Dual3 x2y2 = x2 + y2;
  const Dual3 inv = dconst(1.0f) / (x2y2 + z * z);
  const Dual3 b = datan2(xy_len, z) / xy_len / x2y2;
  const Dual3 a = z * inv / x2y2;
  const Dual3 Jd[6] = {fx * (x2 * a + y2 * b), fx * xy * (a - b), dconst(0.0f) - fx * x * inv,
                       fy * xy * (a - b),      fy * (y2 * a + x2 * b), dconst(0.0f) - fy * y * inv};
  float J[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) J[i] = Jd[i].v;
#pragma unroll
  for (int ia = 0; ia < 3; ++ia)
#pragma unroll
    for (int ib = 0; ib < 3; ++ib) {
      float acc = 0.0f;
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc += J[r * 3 + ia] * v_cov2d[r * 2 + c] * J[c * 3 + ib];
      v_cov3d.v[ia * 3 + ib] = acc;
    }
  float v_J[6];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ia = 0; ia < 3; ++ia) {
      float left = 0.0f, right = 0.0f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int ib = 0; ib < 3; ++ib) {
          left += v_cov2d[r * 2 + c] * J[c * 3 + ib] * cov3d.v[ia * 3 + ib];
          right += v_cov2d[c * 2 + r] * J[c * 3 + ib] * cov3d.v[ib * 3 + ia];
        }
      v_J[r * 3 + ia] = left + right;
    }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    float acc = v_mean2d[0] * m2x.d[k] + v_mean2d[1] * m2y.d[k];
#pragma unroll
    for (int i = 0; i < 6; ++i) acc += v_J[i] * Jd[i].d[k];
    v_mc[k] += acc;
  }
}

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
// with o = sigmoid(logits) (v_opac null: zeros). With v_opac_rows (packed
// layout) the opacity cotangent is per visible pair instead: its sum over
// the Gaussian's pairs (in camera order) takes v_opac's place, and
// v_viewspace (packed layout, if non-null) receives each (camera, Gaussian)
// pair's means2d cotangent densely, zero where the pair has no row.
// PK: the packed layout's per-row opacity cotangent and dense viewspace
// gradient are read / written (a separate instantiation: the two extra
// arguments' registers would cost the others a wave per SIMD).
template <bool ACT, bool PK = false>
__global__ void __launch_bounds__(kProjBlock) projection_bwd_kernel(
    const float* __restrict__ means, const float* __restrict__ covars, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ viewmats, const float* __restrict__ Ks, int64_t C,
    int64_t N, gsplat_projection_params p, const int32_t* __restrict__ radii, const float* __restrict__ conics,
    const float* __restrict__ compensations, const float* __restrict__ v_means2d,
    const float* __restrict__ v_depths, const float* __restrict__ v_conics,
    const float* __restrict__ v_compensations, float* __restrict__ v_means, float* __restrict__ v_covars,
    float* __restrict__ v_quats, float* __restrict__ v_scales, float* __restrict__ vm_partials,
    const float* __restrict__ logits, const float* __restrict__ v_opac, float* __restrict__ v_logits,
    const uint64_t* __restrict__ pmask, const int32_t* __restrict__ pprefix, const float* __restrict__ v_opac_rows,
    float* __restrict__ v_viewspace) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kProjBlock + threadIdx.x;
  const int64_t b = blockIdx.y;
  const bool in_range = n < N;
  const int64_t g = b * N + (in_range ? n : 0);

  // The Gaussian's inputs, then (in the camera loop) its pair's, are loaded
  // before the first wait: a culled pair's loads are wasted, but the
  // backward no longer waits for one round trip to memory after another
  // (the packed layout's step: 1.000 -> 0.983 ms at a million Gaussians).
  const bool use_covars = !ACT && p.use_covars;  // the activated form takes quaternions and log-scales
  float mw[3] = {0.0f, 0.0f, 0.0f};
  float qr[4] = {1.0f, 0.0f, 0.0f, 0.0f};
  float sr[3] = {ACT ? 0.0f : 1.0f, ACT ? 0.0f : 1.0f, ACT ? 0.0f : 1.0f};
  float cv[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  float logit = 0.0f, vop = 0.0f;
  if (in_range) {
    mw[0] = means[g * 3];
    mw[1] = means[g * 3 + 1];
    mw[2] = means[g * 3 + 2];
    if (use_covars) {
#pragma unroll
      for (int k = 0; k < 6; ++k) cv[k] = covars[g * 6 + k];
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) qr[k] = quats[g * 4 + k];
#pragma unroll
      for (int k = 0; k < 3; ++k) sr[k] = scales[g * 3 + k];
    }
    if constexpr (ACT) {
      if (v_logits) logit = logits[g];
      if (v_opac && !(PK && v_opac_rows)) vop = v_opac[g];
    }
  }
  float q[4] = {1.0f, 0.0f, 0.0f, 0.0f};
  float s[3] = {1.0f, 1.0f, 1.0f};
  Mat3 cw;
#pragma unroll
  for (int i = 0; i < 9; ++i) cw.v[i] = 0.0f;
  bool have_cw = false;

  float v_mw_total[3] = {0.0f, 0.0f, 0.0f};
  float v_opac_sum = 0.0f;  // v_opac_rows over the Gaussian's pairs
  Mat3 v_cw_total;
#pragma unroll
  for (int i = 0; i < 9; ++i) v_cw_total.v[i] = 0.0f;

  // one pair's inputs
  struct PairIn {
    float cn[3], vc[3], vm2[2], vdep, comp, vcomp;
  };
  auto load_pair = [&](int64_t idx, PairIn& in) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      in.cn[k] = conics[idx * 3 + k];
      in.vc[k] = v_conics[idx * 3 + k];
    }
    in.vm2[0] = v_means2d[idx * 2];
    in.vm2[1] = v_means2d[idx * 2 + 1];
    in.vdep = v_depths ? v_depths[idx] : 0.0f;
    in.comp = v_compensations ? compensations[idx] : 0.0f;
    in.vcomp = v_compensations ? v_compensations[idx] : 0.0f;
  };

  for (int64_t c = 0; c < C; ++c) {
    const int64_t cam = b * C + c;
    int64_t idx = cam * N + n;
    bool valid;
    PairIn in = {};
    if (pmask) {
      // packed layout: the pair's bit, and its row among the packed pairs
      // (prefix of its 64-pair word + set bits below it)
      valid = false;
      if (in_range) {
        const uint64_t w = pmask[idx >> 6];
        const int bit = static_cast<int>(idx & 63);
        valid = (w >> bit) & 1ull;
        idx = static_cast<int64_t>(pprefix[idx >> 6]) + __popcll(w & ((1ull << bit) - 1ull));
      }
      // the dense viewspace proxy's gradient: this pair's means2d cotangent,
      // zero for a pair without a row
      if (PK && v_viewspace && in_range) {
        float vx = 0.0f, vy = 0.0f;
        if (valid) {
          vx = v_means2d[idx * 2];
          vy = v_means2d[idx * 2 + 1];
        }
        const int64_t slot = cam * N + n;
        v_viewspace[slot * 2] = vx;
        v_viewspace[slot * 2 + 1] = vy;
      }
      if (valid) load_pair(idx, in);
    } else {
      int32_t rx = 0, ry = 0;
      if (in_range) {
        rx = radii[idx * 2];
        ry = radii[idx * 2 + 1];
        load_pair(idx, in);
      }
      valid = in_range && rx > 0 && ry > 0;
    }
    if (!have_cw) {  // once, behind the first pair's loads
      have_cw = true;
      if (use_covars) {
        cw = read_covar(cv);
      } else {
        quat_scale_of<ACT>(qr, sr, q, s);
        cw = covar_from_quat_scale(q, s);
      }
      if (!in_range) {
#pragma unroll
        for (int i = 0; i < 9; ++i) cw.v[i] = 0.0f;
      }
    }
    float vm_part[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) vm_part[i] = 0.0f;
    if (valid) {
      if constexpr (ACT && PK) {
        if (v_opac_rows) v_opac_sum += v_opac_rows[idx];
      }
      const CamFrame f = load_camera(viewmats + cam * 16, Ks + cam * 9);
      const float* cn = in.cn;
      const float* vc = in.vc;
      const float inv[4] = {cn[0], cn[1], cn[1], cn[2]};
      const float vinv[4] = {vc[0], 0.5f * vc[1], 0.5f * vc[1], vc[2]};
      const float tmp[4] = {inv[0] * vinv[0] + inv[1] * vinv[2], inv[0] * vinv[1] + inv[1] * vinv[3],
                            inv[2] * vinv[0] + inv[3] * vinv[2], inv[2] * vinv[1] + inv[3] * vinv[3]};
      float v_cov2d[4] = {-(tmp[0] * inv[0] + tmp[1] * inv[2]), -(tmp[0] * inv[1] + tmp[1] * inv[3]),
                          -(tmp[2] * inv[0] + tmp[3] * inv[2]), -(tmp[2] * inv[1] + tmp[3] * inv[3])};
      if (v_compensations) add_blur_vjp(p.eps2d, inv, in.comp, in.vcomp, v_cov2d);
      float mc[3];
      world_to_cam(f, mw, mc);
      const Mat3 cc = mat3_mul(mat3_mul(f.R, cw), mat3_tr(f.R));
      float v_mc[3] = {0.0f, 0.0f, in.vdep};
      const float vm2[2] = {in.vm2[0], in.vm2[1]};
      Mat3 v_cc;
      if (p.camera_model == 1)
        ortho_proj_vjp(f, v_cov2d, vm2, v_mc, v_cc);
      else if (p.camera_model == 2)
        fisheye_proj_vjp(mc, cc, f, v_cov2d, vm2, v_mc, v_cc);
      else
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
  if (!have_cw && !use_covars) quat_scale_of<ACT>(qr, sr, q, s);  // no camera
#pragma unroll
  for (int i = 0; i < 3; ++i) v_means[g * 3 + i] = v_mw_total[i];
  if (use_covars) {
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
      float vr[4];
      activate_quat_vjp(qr, vq, vr);
#pragma unroll
      for (int i = 0; i < 4; ++i) vq[i] = vr[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) vs[i] = vs[i] * s[i];  // d exp(x) / dx = exp(x)
      if (v_logits) {
        const float o = sigmoid_of(logit);
        if (PK && v_opac_rows)
          v_logits[g] = (v_opac_sum * (1.0f - o)) * o;
        else
          v_logits[g] = v_opac ? (vop * (1.0f - o)) * o : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v_quats[g * 4 + i] = vq[i];
#pragma unroll
    for (int i = 0; i < 3; ++i) v_scales[g * 3 + i] = vs[i];
  }
}

}  // namespace

void launch_projection_bwd(bool act, dim3 grid, hipStream_t s, const float* means, const float* covars,
                           const float* quats, const float* scales, const float* viewmats, const float* Ks, int64_t C,
                           int64_t N, const gsplat_projection_params& p, const int32_t* radii, const float* conics,
                           const float* compensations, const float* v_means2d, const float* v_depths,
                           const float* v_conics, const float* v_compensations, float* v_means, float* v_covars,
                           float* v_quats, float* v_scales, float* vm_partials, const float* logits,
                           const float* v_opac, float* v_logits, const uint64_t* pmask,
                           const int32_t* pprefix, const float* v_opac_rows, float* v_viewspace) {
  if (act && (v_opac_rows || v_viewspace))
    projection_bwd_kernel<true, true><<<grid, kProjBlock, 0, s>>>(
        means, covars, quats, scales, viewmats, Ks, C, N, p, radii, conics, compensations, v_means2d, v_depths,
        v_conics, v_compensations, v_means, v_covars, v_quats, v_scales, vm_partials, logits, v_opac, v_logits, pmask,
        pprefix, v_opac_rows, v_viewspace);
  else if (act)
    projection_bwd_kernel<true><<<grid, kProjBlock, 0, s>>>(means, covars, quats, scales, viewmats, Ks, C, N, p, radii,
                                                            conics, compensations, v_means2d, v_depths, v_conics,
                                                            v_compensations, v_means, v_covars, v_quats, v_scales,
                                                            vm_partials, logits, v_opac, v_logits, pmask, pprefix,
                                                            nullptr, nullptr);
  else
    projection_bwd_kernel<false><<<grid, kProjBlock, 0, s>>>(means, covars, quats, scales, viewmats, Ks, C, N, p,
                                                             radii, conics, compensations, v_means2d, v_depths,
                                                             v_conics, v_compensations, v_means, v_covars, v_quats,
                                                             v_scales, vm_partials, nullptr, nullptr, nullptr, pmask,
                                                             pprefix, nullptr, nullptr);
}

}  // namespace gsplat_hip
