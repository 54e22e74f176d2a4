// gsplat_oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A plain C++ restatement of the reference gsplat_core CPU evaluation loops
// (the `eval_cpu` bodies of a1091150/gsplat-mlx), single-threaded as the
// reference's (OpenMP pragmas split the per-element and per-tile loops only
// when it is compiled with -fopenmp, which the CPU-baseline build of
// bench.py does and the tests' build does not). It exists
// to check the HIP implementation; nothing on the product path may link,
// load or call it. Only tests/, __graft_entry__.smoke() and bench.py's
// CPU-baseline leg use it, always as the reference the GPU results are
// compared with.
//
// Every routine is a template over the scalar type so that the float32
// instantiation reproduces the reference's fp32 arithmetic and the float64
// instantiation serves float64 finite-difference checks of each backward.
//
// Deliberate deviations from the reference CPU loops (each follows the
// reference GPU kernel, whose semantics the reference training path uses):
//   * projection forward culling follows gsplat_projection.metal:249-326
//     (radius clip culls only when BOTH radii <= clip; off-screen cull;
//     orthographic and fisheye camera models), not gsplat_projection.cpp:
//     918-962;
//   * the exclusive scan and the sort replace mx::cumsum / mx::argsort
//     (gsplat_intersect.cpp:207-210, 282-285) with a sequential exclusive
//     scan and std::stable_sort (ties keep encode order).
//
// Parity pins (what checks each function; details in tests/test_oracle_*.py):
//   quat_scale_to_covar fwd  : test.cpp:1723-1757, 1832-1876 known answers,
//                              R orthonormality / closed form R diag(s^2) R^T
//   quat_scale_to_covar bwd  : test.cpp:1920-1951 closed forms, float64 FD
//   projection fwd           : test.cpp:60-130 closed-form pinhole oracle,
//                              test.cpp:352-437 culling cases, textbook EWA
//   projection bwd (+viewmat): float64 FD of the forward
//   spherical_harmonics fwd  : test.cpp:1420-1457 closed forms, scipy real SH
//   spherical_harmonics bwd  : test.cpp:1608-1613 closed form, float64 FD
//   isect count/encode/sort/offset : test.cpp:705-1062 exact integers,
//                              brute-force invariants
//   rasterize fwd            : test.cpp:1111-1131, 1240-1268 closed forms,
//                              brute-force compositing in float64
//   rasterize bwd            : float64 FD of the forward, closed-form v_bg
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <vector>
#if defined(__x86_64__)
#include <xmmintrin.h>
#endif

#ifdef _OPENMP
#include <omp.h>
#include <parallel/algorithm>
#define ORACLE_PRAGMA(x) _Pragma(#x)
// loop iterations run on the OpenMP threads; with cond false, serially
#define ORACLE_PARALLEL_FOR_IF(cond) ORACLE_PRAGMA(omp parallel for schedule(dynamic, 256) if(cond))
#define ORACLE_PARALLEL_TILES ORACLE_PRAGMA(omp parallel for collapse(3) schedule(dynamic, 1))
#define ORACLE_ATOMIC ORACLE_PRAGMA(omp atomic)
#else
#define ORACLE_PARALLEL_FOR_IF(cond)
#define ORACLE_PARALLEL_TILES
#define ORACLE_ATOMIC
#endif
#define ORACLE_PARALLEL_FOR ORACLE_PARALLEL_FOR_IF(true)

namespace {

constexpr float kAlphaThreshold = 1.0f / 255.0f;  // gsplat_projection.cpp:63
constexpr float kGaussianExtend = 3.33f;           // gsplat_projection.cpp:64
constexpr float kMinCompensation = 0.005f;         // gsplat_projection.cpp:65
constexpr float kMaxAlpha = 0.99f;                 // gsplat_rasterize.cpp:24
constexpr float kTransmittanceThreshold = 1.0e-4f; // gsplat_rasterize.cpp:25
constexpr float kMinOneMinusAlpha = 1.0e-6f;       // gsplat_rasterize.cpp:26

template <typename T>
struct M3 {
  T v[9];
};
template <typename T>
struct V3 {
  T v[3];
};

template <typename T>
M3<T> mul(const M3<T>& a, const M3<T>& b) {
  M3<T> o = {};
  for (int r = 0; r < 3; ++r)
    for (int c = 0; c < 3; ++c)
      for (int k = 0; k < 3; ++k) o.v[r * 3 + c] += a.v[r * 3 + k] * b.v[k * 3 + c];
  return o;
}

template <typename T>
M3<T> tr(const M3<T>& a) {
  return M3<T>{{a.v[0], a.v[3], a.v[6], a.v[1], a.v[4], a.v[7], a.v[2], a.v[5], a.v[8]}};
}

// ---------------------------------------------------------------------------
// quaternion (wxyz) -> rotation, gsplat_quat_scale_to_covar.cpp:103-138.
template <typename T>
M3<T> quat_to_rotmat(const T* q) {
  T w = q[0], x = q[1], y = q[2], z = q[3];
  const T norm = std::sqrt(w * w + x * x + y * y + z * z);
  w /= norm;
  x /= norm;
  y /= norm;
  z /= norm;
  const T x2 = x * x, y2 = y * y, z2 = z * z;
  const T xy = x * y, xz = x * z, yz = y * z;
  const T wx = w * x, wy = w * y, wz = w * z;
  return M3<T>{{T(1) - T(2) * (y2 + z2), T(2) * (xy - wz), T(2) * (xz + wy),
                T(2) * (xy + wz), T(1) - T(2) * (x2 + z2), T(2) * (yz - wx),
                T(2) * (xz - wy), T(2) * (yz + wx), T(1) - T(2) * (x2 + y2)}};
}

// R diag(s^2) R^T or R diag(s^-2) R^T, gsplat_quat_scale_to_covar.cpp:140-164.
template <typename T>
M3<T> rot_scale_matrix(const M3<T>& r, const T* scale, bool precision) {
  T s[3] = {scale[0], scale[1], scale[2]};
  if (precision) {
    s[0] = T(1) / s[0];
    s[1] = T(1) / s[1];
    s[2] = T(1) / s[2];
  }
  M3<T> o = {};
  for (int row = 0; row < 3; ++row)
    for (int col = 0; col < 3; ++col) {
      T value = 0;
      for (int k = 0; k < 3; ++k) value += r.v[row * 3 + k] * s[k] * s[k] * r.v[col * 3 + k];
      o.v[row * 3 + col] = value;
    }
  return o;
}

// triu order xx, xy, xz, yy, yz, zz, gsplat_quat_scale_to_covar.cpp:166-179.
template <typename T>
void write_matrix(const M3<T>& m, bool triu, T* out) {
  if (triu) {
    out[0] = m.v[0];
    out[1] = m.v[1];
    out[2] = m.v[2];
    out[3] = m.v[4];
    out[4] = m.v[5];
    out[5] = m.v[8];
  } else {
    for (int i = 0; i < 9; ++i) out[i] = m.v[i];
  }
}

// triu cotangent -> symmetric matrix with halved off-diagonals,
// gsplat_quat_scale_to_covar.cpp:215-236.
template <typename T>
M3<T> cotangent_matrix(bool triu, const T* cot) {
  M3<T> o = {};
  if (triu) {
    o.v[0] = cot[0];
    o.v[1] = T(0.5) * cot[1];
    o.v[2] = T(0.5) * cot[2];
    o.v[3] = T(0.5) * cot[1];
    o.v[4] = cot[3];
    o.v[5] = T(0.5) * cot[4];
    o.v[6] = T(0.5) * cot[2];
    o.v[7] = T(0.5) * cot[4];
    o.v[8] = cot[5];
  } else {
    for (int i = 0; i < 9; ++i) o.v[i] = cot[i];
  }
  return o;
}

// gsplat_quat_scale_to_covar.cpp:238-276.
template <typename T>
void quat_to_rotmat_vjp_qs(const T* quat, const M3<T>& v_r, T* v_quat) {
  T w = quat[0], x = quat[1], y = quat[2], z = quat[3];
  const T norm = std::sqrt(w * w + x * x + y * y + z * z);
  const T inv_norm = T(1) / norm;
  w *= inv_norm;
  x *= inv_norm;
  y *= inv_norm;
  z *= inv_norm;
  const T* g = v_r.v;
  T n[4] = {};
  n[1] = T(2) * y * g[1] + T(2) * z * g[2] + T(2) * y * g[3] - T(4) * x * g[4] -
         T(2) * w * g[5] + T(2) * z * g[6] + T(2) * w * g[7] - T(4) * x * g[8];
  n[2] = -T(4) * y * g[0] + T(2) * x * g[1] + T(2) * w * g[2] + T(2) * x * g[3] +
         T(2) * z * g[5] - T(2) * w * g[6] + T(2) * z * g[7] - T(4) * y * g[8];
  n[3] = -T(4) * z * g[0] - T(2) * w * g[1] + T(2) * x * g[2] + T(2) * w * g[3] -
         T(4) * z * g[4] + T(2) * y * g[5] + T(2) * x * g[6] + T(2) * y * g[7];
  n[0] = -T(2) * z * g[1] + T(2) * y * g[2] + T(2) * z * g[3] - T(2) * x * g[5] -
         T(2) * y * g[6] + T(2) * x * g[7];
  const T dot = n[0] * w + n[1] * x + n[2] * y + n[3] * z;
  v_quat[0] += (n[0] - dot * w) * inv_norm;
  v_quat[1] += (n[1] - dot * x) * inv_norm;
  v_quat[2] += (n[2] - dot * y) * inv_norm;
  v_quat[3] += (n[3] - dot * z) * inv_norm;
}

// gsplat_quat_scale_to_covar.cpp:278-333.
template <typename T>
void quat_scale_vjp(const T* quat, const T* scale, const M3<T>& r, const M3<T>& v_matrix,
                    bool precision, T* v_quat, T* v_scale) {
  T s[3] = {scale[0], scale[1], scale[2]};
  if (precision) {
    s[0] = T(1) / s[0];
    s[1] = T(1) / s[1];
    s[2] = T(1) / s[2];
  }
  M3<T> m = {};
  for (int row = 0; row < 3; ++row)
    for (int col = 0; col < 3; ++col) m.v[row * 3 + col] = r.v[row * 3 + col] * s[col];
  M3<T> v_m = {};
  for (int row = 0; row < 3; ++row)
    for (int col = 0; col < 3; ++col) {
      T value = 0;
      for (int k = 0; k < 3; ++k)
        value += (v_matrix.v[row * 3 + k] + v_matrix.v[k * 3 + row]) * m.v[k * 3 + col];
      v_m.v[row * 3 + col] = value;
    }
  M3<T> v_r = {};
  for (int row = 0; row < 3; ++row)
    for (int col = 0; col < 3; ++col) v_r.v[row * 3 + col] = v_m.v[row * 3 + col] * s[col];
  quat_to_rotmat_vjp_qs(quat, v_r, v_quat);
  for (int col = 0; col < 3; ++col) {
    T grad = 0;
    for (int row = 0; row < 3; ++row) grad += r.v[row * 3 + col] * v_m.v[row * 3 + col];
    if (precision)
      v_scale[col] += -s[col] * s[col] * grad;
    else
      v_scale[col] += grad;
  }
}

// GSPlatQuatScaleToCovarPreci::eval_cpu, gsplat_quat_scale_to_covar.cpp:374-405.
template <typename T>
void qs_forward(const T* quats, const T* scales, int64_t n, int compute_covar, int compute_preci,
                int triu, T* covars, T* precis) {
  const int stride = triu ? 6 : 9;
  ORACLE_PARALLEL_FOR
  for (int64_t e = 0; e < n; ++e) {
    const M3<T> r = quat_to_rotmat(quats + e * 4);
    if (compute_covar) write_matrix(rot_scale_matrix(r, scales + e * 3, false), triu != 0, covars + e * stride);
    if (compute_preci) write_matrix(rot_scale_matrix(r, scales + e * 3, true), triu != 0, precis + e * stride);
  }
}

// GSPlatQuatScaleToCovarPreciBackward::eval_cpu, gsplat_quat_scale_to_covar.cpp:407-468.
template <typename T>
void qs_backward(const T* quats, const T* scales, const T* v_covars, const T* v_precis, int64_t n,
                 int triu, T* v_quats, T* v_scales) {
  const int stride = triu ? 6 : 9;
  ORACLE_PARALLEL_FOR
  for (int64_t e = 0; e < n; ++e) {
    T vq[4] = {}, vs[3] = {};
    const M3<T> r = quat_to_rotmat(quats + e * 4);
    if (v_covars) quat_scale_vjp(quats + e * 4, scales + e * 3, r, cotangent_matrix(triu != 0, v_covars + e * stride), false, vq, vs);
    if (v_precis) quat_scale_vjp(quats + e * 4, scales + e * 3, r, cotangent_matrix(triu != 0, v_precis + e * stride), true, vq, vs);
    for (int i = 0; i < 4; ++i) v_quats[e * 4 + i] = vq[i];
    for (int i = 0; i < 3; ++i) v_scales[e * 3 + i] = vs[i];
  }
}

// ---------------------------------------------------------------------------
// Projection.

struct ProjParams {
  int32_t image_width;
  int32_t image_height;
  float eps2d;
  float near_plane;
  float far_plane;
  float radius_clip;
  int32_t calc_compensations;
  int32_t camera_model;
  int32_t use_covars;
  int32_t use_opacities;
};

template <typename T>
M3<T> read_covar(const T* c) {
  return M3<T>{{c[0], c[1], c[2], c[1], c[3], c[4], c[2], c[4], c[5]}};
}

// gsplat_projection.cpp:204-218 (M M^T with M = R diag(s)).
template <typename T>
M3<T> covar_from_quat_scale(const T* quat, const T* scale) {
  const M3<T> r = quat_to_rotmat(quat);
  M3<T> o = {};
  for (int row = 0; row < 3; ++row)
    for (int col = 0; col < 3; ++col) {
      T value = 0;
      for (int k = 0; k < 3; ++k) value += r.v[row * 3 + k] * scale[k] * scale[k] * r.v[col * 3 + k];
      o.v[row * 3 + col] = value;
    }
  return o;
}

template <typename T>
M3<T> view_rotation(const T* view) {
  return M3<T>{{view[0], view[1], view[2], view[4], view[5], view[6], view[8], view[9], view[10]}};
}

// 2x3 Jacobian J and mean2d for the three camera models,
// gsplat_projection.metal:122-200 (pinhole also gsplat_projection.cpp:486-499).
template <typename T>
void camera_jacobian(int model, const T* mc, T fx, T fy, T cx, T cy, int width, int height,
                     T* J, T* mean2d) {
  const T x = mc[0], y = mc[1], z = mc[2];
  if (model == 1) {  // orthographic, gsplat_projection.metal:153-168
    J[0] = fx; J[1] = 0; J[2] = 0;
    J[3] = 0; J[4] = fy; J[5] = 0;
    mean2d[0] = fx * x + cx;
    mean2d[1] = fy * y + cy;
    return;
  }
  if (model == 2) {  // fisheye, gsplat_projection.metal:170-200
    const T eps = T(0.0000001);
    const T xy_len = std::sqrt(x * x + y * y) + eps;
    const T theta = std::atan2(xy_len, z + eps);
    mean2d[0] = x * fx * theta / xy_len + cx;
    mean2d[1] = y * fy * theta / xy_len + cy;
    const T x2 = x * x + eps;
    const T y2 = y * y;
    const T xy = x * y;
    const T x2y2 = x2 + y2;
    const T x2y2z2_inv = T(1) / (x2y2 + z * z);
    const T b = std::atan2(xy_len, z) / xy_len / x2y2;
    const T a = z * x2y2z2_inv / x2y2;
    J[0] = fx * (x2 * a + y2 * b);
    J[1] = fx * xy * (a - b);
    J[2] = -fx * x * x2y2z2_inv;
    J[3] = fy * xy * (a - b);
    J[4] = fy * (y2 * a + x2 * b);
    J[5] = -fy * y * x2y2z2_inv;
    return;
  }
  const T tan_fovx = T(0.5) * T(width) / fx;
  const T tan_fovy = T(0.5) * T(height) / fy;
  const T lim_x_pos = (T(width) - cx) / fx + T(0.3) * tan_fovx;
  const T lim_x_neg = cx / fx + T(0.3) * tan_fovx;
  const T lim_y_pos = (T(height) - cy) / fy + T(0.3) * tan_fovy;
  const T lim_y_neg = cy / fy + T(0.3) * tan_fovy;
  const T rz = T(1) / z;
  const T rz2 = rz * rz;
  const T tx = z * std::min(lim_x_pos, std::max(-lim_x_neg, x * rz));
  const T ty = z * std::min(lim_y_pos, std::max(-lim_y_neg, y * rz));
  J[0] = fx * rz; J[1] = 0; J[2] = -fx * tx * rz2;
  J[3] = 0; J[4] = fy * rz; J[5] = -fy * ty * rz2;
  mean2d[0] = fx * x * rz + cx;
  mean2d[1] = fy * y * rz + cy;
}

// Forward projection with GPU culling semantics, gsplat_projection.metal:214-339
// (per-Gaussian math as gsplat_projection.cpp:446-521).
template <typename T>
void proj_forward(const T* means, const T* covars, const T* quats, const T* scales,
                  const T* opacities, const T* viewmats, const T* Ks, int64_t B, int64_t C,
                  int64_t N, const ProjParams& p, int32_t* radii, T* means2d, T* depths, T* conics,
                  T* compensations) {
  const int64_t total = B * C * N;
  std::memset(radii, 0, sizeof(int32_t) * total * 2);
  std::memset(means2d, 0, sizeof(T) * total * 2);
  std::memset(depths, 0, sizeof(T) * total);
  std::memset(conics, 0, sizeof(T) * total * 3);
  if (p.calc_compensations) std::memset(compensations, 0, sizeof(T) * total);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      ORACLE_PARALLEL_FOR
      for (int64_t n = 0; n < N; ++n) {
        const int64_t idx = (b * C + c) * N + n;
        const int64_t g = b * N + n;
        const T* view = viewmats + (b * C + c) * 16;
        const T* K = Ks + (b * C + c) * 9;
        const M3<T> R = view_rotation(view);
        const T* mw = means + g * 3;
        const T mc[3] = {R.v[0] * mw[0] + R.v[1] * mw[1] + R.v[2] * mw[2] + view[3],
                         R.v[3] * mw[0] + R.v[4] * mw[1] + R.v[5] * mw[2] + view[7],
                         R.v[6] * mw[0] + R.v[7] * mw[1] + R.v[8] * mw[2] + view[11]};
        if (mc[2] < T(p.near_plane) || mc[2] > T(p.far_plane)) continue;
        const M3<T> cw = p.use_covars ? read_covar(covars + g * 6)
                                      : covar_from_quat_scale(quats + g * 4, scales + g * 3);
        const M3<T> cc = mul(mul(R, cw), tr(R));
        T J[6], m2[2];
        camera_jacobian(p.camera_model, mc, K[0], K[4], K[2], K[5], p.image_width, p.image_height, J, m2);
        T cov2d[4] = {};
        for (int row = 0; row < 2; ++row)
          for (int col = 0; col < 2; ++col)
            for (int a = 0; a < 3; ++a)
              for (int bb = 0; bb < 3; ++bb)
                cov2d[row * 2 + col] += J[row * 3 + a] * cc.v[a * 3 + bb] * J[col * 3 + bb];
        // add_blur, gsplat_projection.metal:202-212
        const T det_orig = cov2d[0] * cov2d[3] - cov2d[1] * cov2d[2];
        cov2d[0] += T(p.eps2d);
        cov2d[3] += T(p.eps2d);
        const T det = cov2d[0] * cov2d[3] - cov2d[1] * cov2d[2];
        const T comp = std::sqrt(std::max(T(kMinCompensation) * T(kMinCompensation), det_orig / det));
        if (det <= T(0)) continue;
        const T inv_det = T(1) / det;
        T extend = T(kGaussianExtend);
        if (p.use_opacities) {
          T op = opacities[g];
          if (p.calc_compensations) op *= comp;
          if (op < T(kAlphaThreshold)) continue;
          extend = std::min(T(kGaussianExtend), std::sqrt(T(2) * std::log(op / T(kAlphaThreshold))));
        }
        const T rx = std::ceil(extend * std::sqrt(cov2d[0]));
        const T ry = std::ceil(extend * std::sqrt(cov2d[3]));
        if (rx <= T(p.radius_clip) && ry <= T(p.radius_clip)) continue;
        if (m2[0] + rx <= T(0) || m2[0] - rx >= T(p.image_width) || m2[1] + ry <= T(0) ||
            m2[1] - ry >= T(p.image_height))
          continue;
        radii[idx * 2] = static_cast<int32_t>(rx);
        radii[idx * 2 + 1] = static_cast<int32_t>(ry);
        means2d[idx * 2] = m2[0];
        means2d[idx * 2 + 1] = m2[1];
        depths[idx] = mc[2];
        conics[idx * 3] = cov2d[3] * inv_det;
        conics[idx * 3 + 1] = -cov2d[1] * inv_det;
        conics[idx * 3 + 2] = cov2d[0] * inv_det;
        if (p.calc_compensations) compensations[idx] = comp;
      }
}

// gsplat_projection.cpp:262-284.
template <typename T>
void add_blur_vjp(T eps2d, const T* conic_blur, T compensation, T v_compensation, T* v_covar) {
  const T det_conic_blur = conic_blur[0] * conic_blur[3] - conic_blur[1] * conic_blur[2];
  const T v_sqr_comp = v_compensation * T(0.5) / (compensation + T(1.0e-6));
  const T one_minus_sqr_comp = T(1) - compensation * compensation;
  v_covar[0] += v_sqr_comp * (one_minus_sqr_comp * conic_blur[0] - eps2d * det_conic_blur);
  v_covar[1] += v_sqr_comp * (one_minus_sqr_comp * conic_blur[1]);
  v_covar[2] += v_sqr_comp * (one_minus_sqr_comp * conic_blur[2]);
  v_covar[3] += v_sqr_comp * (one_minus_sqr_comp * conic_blur[3] - eps2d * det_conic_blur);
}

// gsplat_projection.cpp:286-377.
// Orthographic camera (upstream gsplat's ortho_proj_vjp; the reference has
// the forward only, its backward is guarded at gsplat_projection.cpp:157-160):
// J = [[fx, 0, 0], [0, fy, 0]] does not depend on the mean, so
// v_cov3d = J^T v_cov2d J and v_mean3d += (fx v_mean2d.x, fy v_mean2d.y, 0).
template <typename T>
void ortho_proj_vjp(T fx, T fy, const T* v_cov2d, const T* v_mean2d, T* v_mean3d, M3<T>& v_cov3d) {
  const T J[6] = {fx, T(0), T(0), T(0), fy, T(0)};
  for (int a = 0; a < 3; ++a)
    for (int b = 0; b < 3; ++b) {
      T acc = 0;
      for (int r = 0; r < 2; ++r)
        for (int c = 0; c < 2; ++c) acc += J[r * 3 + a] * v_cov2d[r * 2 + c] * J[c * 3 + b];
      v_cov3d.v[a * 3 + b] = acc;
    }
  v_mean3d[0] += fx * v_mean2d[0];
  v_mean3d[1] += fy * v_mean2d[1];
}

// Equidistant fisheye (upstream gsplat's fisheye_proj_vjp; forward only in
// the reference): the image point and J are differentiated as forward-mode
// dual numbers (value and d/dx, d/dy, d/dz) through the forward's formulas
// (camera_jacobian above), eps terms included. Pinned by float64 finite
// differences of the fisheye forward.
template <typename T>
struct Dual {
  T v, d[3];
};
template <typename T>
Dual<T> dc(T c) { return {c, {T(0), T(0), T(0)}}; }
template <typename T>
Dual<T> operator+(const Dual<T>& a, const Dual<T>& b) {
  return {a.v + b.v, {a.d[0] + b.d[0], a.d[1] + b.d[1], a.d[2] + b.d[2]}};
}
template <typename T>
Dual<T> operator-(const Dual<T>& a, const Dual<T>& b) {
  return {a.v - b.v, {a.d[0] - b.d[0], a.d[1] - b.d[1], a.d[2] - b.d[2]}};
}
template <typename T>
Dual<T> operator*(const Dual<T>& a, const Dual<T>& b) {
  return {a.v * b.v, {a.d[0] * b.v + a.v * b.d[0], a.d[1] * b.v + a.v * b.d[1], a.d[2] * b.v + a.v * b.d[2]}};
}
template <typename T>
Dual<T> operator/(const Dual<T>& a, const Dual<T>& b) {
  const T q = a.v / b.v;
  return {q, {(a.d[0] - q * b.d[0]) / b.v, (a.d[1] - q * b.d[1]) / b.v, (a.d[2] - q * b.d[2]) / b.v}};
}
template <typename T>
Dual<T> dsqrt(const Dual<T>& a) {
  const T r = std::sqrt(a.v);
  return {r, {a.d[0] / (T(2) * r), a.d[1] / (T(2) * r), a.d[2] / (T(2) * r)}};
}
template <typename T>
Dual<T> datan2(const Dual<T>& u, const Dual<T>& w) {
  const T den = u.v * u.v + w.v * w.v;
  Dual<T> o;
  o.v = std::atan2(u.v, w.v);
  for (int k = 0; k < 3; ++k) o.d[k] = (w.v * u.d[k] - u.v * w.d[k]) / den;
  return o;
}

template <typename T>
void fisheye_proj_vjp(const T* mc, const M3<T>& cov3d, T fx_, T fy_, const T* v_cov2d, const T* v_mean2d,
                      T* v_mean3d, M3<T>& v_cov3d) {
  const Dual<T> x = {mc[0], {T(1), T(0), T(0)}}, y = {mc[1], {T(0), T(1), T(0)}}, z = {mc[2], {T(0), T(0), T(1)}};
  const Dual<T> eps = dc(T(0.0000001f)), fx = dc(fx_), fy = dc(fy_);
  const Dual<T> xy_len = dsqrt(x * x + y * y) + eps;
  const Dual<T> theta = datan2(xy_len, z + eps);
  const Dual<T> m2[2] = {x * fx * theta / xy_len, y * fy * theta / xy_len};
  const Dual<T> x2 = x * x + eps, y2 = y * y, xy = x * y;
  const Dual<T> x2y2 = x2 + y2;
  const Dual<T> inv = dc(T(1)) / (x2y2 + z * z);
  const Dual<T> b = datan2(xy_len, z) / xy_len / x2y2;
  const Dual<T> a = z * inv / x2y2;
  const Dual<T> J[6] = {fx * (x2 * a + y2 * b), fx * xy * (a - b), dc(T(0)) - fx * x * inv,
                        fy * xy * (a - b),      fy * (y2 * a + x2 * b), dc(T(0)) - fy * y * inv};
  for (int ia = 0; ia < 3; ++ia)
    for (int ib = 0; ib < 3; ++ib) {
      T acc = 0;
      for (int r = 0; r < 2; ++r)
        for (int c = 0; c < 2; ++c) acc += J[r * 3 + ia].v * v_cov2d[r * 2 + c] * J[c * 3 + ib].v;
      v_cov3d.v[ia * 3 + ib] = acc;
    }
  // d/dJ of J cov3d J^T contracted with v_cov2d
  T v_J[6];
  for (int r = 0; r < 2; ++r)
    for (int ia = 0; ia < 3; ++ia) {
      T acc = 0;
      for (int c = 0; c < 2; ++c)
        for (int ib = 0; ib < 3; ++ib)
          acc += v_cov2d[r * 2 + c] * J[c * 3 + ib].v * cov3d.v[ia * 3 + ib] +
                 v_cov2d[c * 2 + r] * J[c * 3 + ib].v * cov3d.v[ib * 3 + ia];
      v_J[r * 3 + ia] = acc;
    }
  for (int k = 0; k < 3; ++k) {
    T acc = v_mean2d[0] * m2[0].d[k] + v_mean2d[1] * m2[1].d[k];
    for (int i = 0; i < 6; ++i) acc += v_J[i] * J[i].d[k];
    v_mean3d[k] += acc;
  }
}

template <typename T>
void persp_proj_vjp(const T* mean3d, const M3<T>& cov3d, T fx, T fy, T cx, T cy, int width,
                    int height, const T* v_cov2d, const T* v_mean2d, T* v_mean3d, M3<T>& v_cov3d) {
  const T x = mean3d[0], y = mean3d[1], z = mean3d[2];
  const T tan_fovx = T(0.5) * T(width) / fx;
  const T tan_fovy = T(0.5) * T(height) / fy;
  const T lim_x_pos = (T(width) - cx) / fx + T(0.3) * tan_fovx;
  const T lim_x_neg = cx / fx + T(0.3) * tan_fovx;
  const T lim_y_pos = (T(height) - cy) / fy + T(0.3) * tan_fovy;
  const T lim_y_neg = cy / fy + T(0.3) * tan_fovy;
  const T rz = T(1) / z;
  const T rz2 = rz * rz;
  const T rz3 = rz2 * rz;
  const T x_rz = x * rz;
  const T y_rz = y * rz;
  const T tx = z * std::min(lim_x_pos, std::max(-lim_x_neg, x_rz));
  const T ty = z * std::min(lim_y_pos, std::max(-lim_y_neg, y_rz));
  const T J[6] = {fx * rz, 0, -fx * tx * rz2, 0, fy * rz, -fy * ty * rz2};
  for (int a = 0; a < 3; ++a)
    for (int b = 0; b < 3; ++b)
      for (int r = 0; r < 2; ++r)
        for (int c = 0; c < 2; ++c)
          v_cov3d.v[a * 3 + b] += J[r * 3 + a] * v_cov2d[r * 2 + c] * J[c * 3 + b];
  v_mean3d[0] += fx * rz * v_mean2d[0];
  v_mean3d[1] += fy * rz * v_mean2d[1];
  v_mean3d[2] += -(fx * x * v_mean2d[0] + fy * y * v_mean2d[1]) * rz2;
  T v_J[6] = {};
  for (int r = 0; r < 2; ++r)
    for (int a = 0; a < 3; ++a) {
      T left = 0, right = 0;
      for (int c = 0; c < 2; ++c)
        for (int b = 0; b < 3; ++b) {
          left += v_cov2d[r * 2 + c] * J[c * 3 + b] * cov3d.v[a * 3 + b];
          right += v_cov2d[c * 2 + r] * J[c * 3 + b] * cov3d.v[b * 3 + a];
        }
      v_J[r * 3 + a] = left + right;
    }
  if (x_rz <= lim_x_pos && x_rz >= -lim_x_neg)
    v_mean3d[0] += -fx * rz2 * v_J[2];
  else
    v_mean3d[2] += -fx * rz3 * tx * v_J[2];
  if (y_rz <= lim_y_pos && y_rz >= -lim_y_neg)
    v_mean3d[1] += -fy * rz2 * v_J[5];
  else
    v_mean3d[2] += -fy * rz3 * ty * v_J[5];
  v_mean3d[2] += -fx * rz2 * v_J[0] - fy * rz2 * v_J[4] + T(2) * fx * tx * rz3 * v_J[2] +
                 T(2) * fy * ty * rz3 * v_J[5];
}

// gsplat_projection.cpp:404-437.
template <typename T>
void quat_to_rotmat_vjp_proj(const T* quat, const M3<T>& v_R, T* v_quat) {
  T w = quat[0], x = quat[1], y = quat[2], z = quat[3];
  const T inv_norm = T(1) / std::sqrt(w * w + x * x + y * y + z * z);
  w *= inv_norm;
  x *= inv_norm;
  y *= inv_norm;
  z *= inv_norm;
  const T* g = v_R.v;
  const T n[4] = {
      T(2) * (x * (g[7] - g[5]) + y * (g[2] - g[6]) + z * (g[3] - g[1])),
      T(2) * (-T(2) * x * (g[4] + g[8]) + y * (g[1] + g[3]) + z * (g[2] + g[6]) + w * (g[7] - g[5])),
      T(2) * (x * (g[1] + g[3]) - T(2) * y * (g[0] + g[8]) + z * (g[5] + g[7]) + w * (g[2] - g[6])),
      T(2) * (x * (g[2] + g[6]) + y * (g[5] + g[7]) - T(2) * z * (g[0] + g[4]) + w * (g[3] - g[1])),
  };
  const T qn[4] = {w, x, y, z};
  T dot = 0;
  for (int i = 0; i < 4; ++i) dot += n[i] * qn[i];
  for (int i = 0; i < 4; ++i) v_quat[i] += (n[i] - dot * qn[i]) * inv_norm;
}

// gsplat_projection.cpp:439-474.
template <typename T>
void quat_scale_to_covar_vjp(const T* quat, const T* scale, const M3<T>& v_covar, T* v_quat, T* v_scale) {
  const M3<T> R = quat_to_rotmat(quat);
  M3<T> M = {};
  for (int row = 0; row < 3; ++row)
    for (int col = 0; col < 3; ++col) M.v[row * 3 + col] = R.v[row * 3 + col] * scale[col];
  M3<T> sym = {};
  for (int r = 0; r < 3; ++r)
    for (int c = 0; c < 3; ++c) sym.v[r * 3 + c] = v_covar.v[r * 3 + c] + v_covar.v[c * 3 + r];
  const M3<T> v_M = mul(sym, M);
  M3<T> v_R = {};
  for (int row = 0; row < 3; ++row)
    for (int col = 0; col < 3; ++col) {
      v_R.v[row * 3 + col] = v_M.v[row * 3 + col] * scale[col];
      v_scale[col] += v_M.v[row * 3 + col] * R.v[row * 3 + col];
    }
  quat_to_rotmat_vjp_proj(quat, v_R, v_quat);
}

// GSPlatProjectionEWA3DGSFusedBackward::eval_cpu, gsplat_projection.cpp:965-1121
// (pinhole only, as the reference).
template <typename T>
void proj_backward(const T* means, const T* covars, const T* quats, const T* scales,
                   const T* viewmats, const T* Ks, int64_t B, int64_t C, int64_t N,
                   const ProjParams& p, const int32_t* radii, const T* conics,
                   const T* compensations, const T* v_means2d, const T* v_depths, const T* v_conics,
                   const T* v_compensations, T* v_means, T* v_covars, T* v_quats, T* v_scales,
                   T* v_viewmats) {
  std::memset(v_means, 0, sizeof(T) * B * N * 3);
  if (p.use_covars) std::memset(v_covars, 0, sizeof(T) * B * N * 6);
  else {
    std::memset(v_quats, 0, sizeof(T) * B * N * 4);
    std::memset(v_scales, 0, sizeof(T) * B * N * 3);
  }
  if (v_viewmats) std::memset(v_viewmats, 0, sizeof(T) * B * C * 16);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      ORACLE_PARALLEL_FOR_IF(v_viewmats == nullptr)  // the view-matrix sums are shared across n
      for (int64_t n = 0; n < N; ++n) {
        const int64_t idx = (b * C + c) * N + n;
        if (radii[idx * 2] <= 0 || radii[idx * 2 + 1] <= 0) continue;
        const int64_t g = b * N + n;
        const T* view = viewmats + (b * C + c) * 16;
        const T* K = Ks + (b * C + c) * 9;
        const T* cn = conics + idx * 3;
        const T* vc = v_conics + idx * 3;
        const T inv[4] = {cn[0], cn[1], cn[1], cn[2]};
        const T vinv[4] = {vc[0], T(0.5) * vc[1], T(0.5) * vc[1], vc[2]};
        // v_cov2d = -inv * vinv * inv
        T tmp[4] = {inv[0] * vinv[0] + inv[1] * vinv[2], inv[0] * vinv[1] + inv[1] * vinv[3],
                    inv[2] * vinv[0] + inv[3] * vinv[2], inv[2] * vinv[1] + inv[3] * vinv[3]};
        T v_cov2d[4] = {-(tmp[0] * inv[0] + tmp[1] * inv[2]), -(tmp[0] * inv[1] + tmp[1] * inv[3]),
                        -(tmp[2] * inv[0] + tmp[3] * inv[2]), -(tmp[2] * inv[1] + tmp[3] * inv[3])};
        if (v_compensations)
          add_blur_vjp(T(p.eps2d), inv, compensations[idx], v_compensations[idx], v_cov2d);
        const M3<T> R = view_rotation(view);
        const T* mw = means + g * 3;
        const T mc[3] = {R.v[0] * mw[0] + R.v[1] * mw[1] + R.v[2] * mw[2] + view[3],
                         R.v[3] * mw[0] + R.v[4] * mw[1] + R.v[5] * mw[2] + view[7],
                         R.v[6] * mw[0] + R.v[7] * mw[1] + R.v[8] * mw[2] + view[11]};
        const M3<T> cw = p.use_covars ? read_covar(covars + g * 6)
                                      : covar_from_quat_scale(quats + g * 4, scales + g * 3);
        const M3<T> cc = mul(mul(R, cw), tr(R));
        T v_mc[3] = {0, 0, v_depths[idx]};
        M3<T> v_cc = {};
        if (p.camera_model == 1)
          ortho_proj_vjp(K[0], K[4], v_cov2d, v_means2d + idx * 2, v_mc, v_cc);
        else if (p.camera_model == 2)
          fisheye_proj_vjp(mc, cc, K[0], K[4], v_cov2d, v_means2d + idx * 2, v_mc, v_cc);
        else
          persp_proj_vjp(mc, cc, K[0], K[4], K[2], K[5], p.image_width, p.image_height, v_cov2d,
                         v_means2d + idx * 2, v_mc, v_cc);
        // pos_w2c_vjp / covar_w2c_vjp, gsplat_projection.cpp:379-402
        M3<T> v_R = {};
        T v_t[3] = {};
        for (int row = 0; row < 3; ++row) {
          v_t[row] += v_mc[row];
          for (int col = 0; col < 3; ++col) v_R.v[row * 3 + col] += v_mc[row] * mw[col];
        }
        T v_mw[3];
        for (int i = 0; i < 3; ++i) v_mw[i] = R.v[0 * 3 + i] * v_mc[0] + R.v[1 * 3 + i] * v_mc[1] + R.v[2 * 3 + i] * v_mc[2];
        const M3<T> term1 = mul(mul(v_cc, R), tr(cw));
        const M3<T> term2 = mul(mul(tr(v_cc), R), cw);
        const M3<T> v_cw = mul(mul(tr(R), v_cc), R);
        for (int i = 0; i < 9; ++i) v_R.v[i] += term1.v[i] + term2.v[i];
        for (int i = 0; i < 3; ++i) v_means[g * 3 + i] += v_mw[i];
        if (p.use_covars) {
          T* o = v_covars + g * 6;
          o[0] += v_cw.v[0];
          o[1] += v_cw.v[1] + v_cw.v[3];
          o[2] += v_cw.v[2] + v_cw.v[6];
          o[3] += v_cw.v[4];
          o[4] += v_cw.v[5] + v_cw.v[7];
          o[5] += v_cw.v[8];
        } else {
          quat_scale_to_covar_vjp(quats + g * 4, scales + g * 3, v_cw, v_quats + g * 4, v_scales + g * 3);
        }
        if (v_viewmats) {
          T* o = v_viewmats + (b * C + c) * 16;
          for (int row = 0; row < 3; ++row) {
            for (int col = 0; col < 3; ++col) o[row * 4 + col] += v_R.v[row * 3 + col];
            o[row * 4 + 3] += v_t[row];
          }
        }
      }
}

// ---------------------------------------------------------------------------
// Spherical harmonics, gsplat_spherical_harmonics.cpp:112-187 (basis values).
template <typename T>
void sh_basis(int degree, const T* dir, T* basis) {
  const int count = (degree + 1) * (degree + 1);
  for (int i = 0; i < count; ++i) basis[i] = 0;
  basis[0] = T(0.2820947917738781);
  if (degree < 1) return;
  const T norm = std::sqrt(dir[0] * dir[0] + dir[1] * dir[1] + dir[2] * dir[2]);
  if (norm == T(0)) return;
  const T x = dir[0] / norm, y = dir[1] / norm, z = dir[2] / norm;
  const T C1 = T(0.48860251190292);
  basis[1] = -C1 * y;
  basis[2] = C1 * z;
  basis[3] = -C1 * x;
  if (degree < 2) return;
  const T z2 = z * z;
  const T f_tmp0_b = T(-1.092548430592079) * z;
  const T f_c1 = x * x - y * y;
  const T f_s1 = T(2) * x * y;
  basis[4] = T(0.5462742152960395) * f_s1;
  basis[5] = f_tmp0_b * y;
  basis[6] = T(0.9461746957575601) * z2 - T(0.3153915652525201);
  basis[7] = f_tmp0_b * x;
  basis[8] = T(0.5462742152960395) * f_c1;
  if (degree < 3) return;
  const T f_tmp0_c = T(-2.285228997322329) * z2 + T(0.4570457994644658);
  const T f_tmp1_b = T(1.445305721320277) * z;
  const T f_c2 = x * f_c1 - y * f_s1;
  const T f_s2 = x * f_s1 + y * f_c1;
  basis[9] = T(-0.5900435899266435) * f_s2;
  basis[10] = f_tmp1_b * f_s1;
  basis[11] = f_tmp0_c * y;
  basis[12] = z * (T(1.865881662950577) * z2 - T(1.119528997770346));
  basis[13] = f_tmp0_c * x;
  basis[14] = f_tmp1_b * f_c1;
  basis[15] = T(-0.5900435899266435) * f_c2;
  if (degree < 4) return;
  const T f_tmp0_d = z * (T(-4.683325804901025) * z2 + T(2.007139630671868));
  const T f_tmp1_c = T(3.31161143515146) * z2 - T(0.47308734787878);
  const T f_tmp2_b = T(-1.770130769779931) * z;
  const T f_c3 = x * f_c2 - y * f_s2;
  const T f_s3 = x * f_s2 + y * f_c2;
  basis[16] = T(0.6258357354491763) * f_s3;
  basis[17] = f_tmp2_b * f_s2;
  basis[18] = f_tmp1_c * f_s1;
  basis[19] = f_tmp0_d * y;
  basis[20] = T(1.984313483298443) * z * basis[12] - T(1.006230589874905) * basis[6];
  basis[21] = f_tmp0_d * x;
  basis[22] = f_tmp1_c * f_c1;
  basis[23] = f_tmp2_b * f_c2;
  basis[24] = T(0.6258357354491763) * f_c3;
}

// GSPlatSphericalHarmonics::eval_cpu, gsplat_spherical_harmonics.cpp:466-501.
// The per-channel accumulation follows sh_channel_to_color
// (gsplat_spherical_harmonics.cpp:189-286): DC term first, then one sum per
// band added to the running result.
template <typename T>
void sh_forward(int degree, const T* dirs, const T* coeffs, const uint8_t* masks, int64_t n,
                int64_t K, T* colors) {
  ORACLE_PARALLEL_FOR
  for (int64_t e = 0; e < n; ++e) {
    T basis[25];
    if (masks && !masks[e]) {
      colors[e * 3] = colors[e * 3 + 1] = colors[e * 3 + 2] = 0;
      continue;
    }
    sh_basis(degree, dirs + e * 3, basis);
    const T* co = coeffs + e * K * 3;
    const T* d = dirs + e * 3;
    const T norm = std::sqrt(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
    for (int ch = 0; ch < 3; ++ch) {
      T result = T(0.2820947917738781) * co[ch];
      if (degree >= 1 && norm != T(0)) {
        const T x = d[0] / norm, y = d[1] / norm, z = d[2] / norm;
        result += T(0.48860251190292) * (-y * co[3 + ch] + z * co[6 + ch] - x * co[9 + ch]);
        for (int l = 2; l <= degree; ++l) {
          T band = basis[l * l] * co[l * l * 3 + ch];
          for (int b = l * l + 1; b < (l + 1) * (l + 1); ++b) band += basis[b] * co[b * 3 + ch];
          result += band;
        }
      }
      colors[e * 3 + ch] = result;
    }
  }
}

// Analytic d(basis)/d(unit dir), then tangent projection,
// gsplat_spherical_harmonics.cpp:288-425.
template <typename T>
void sh_dir_vjp(int degree, const T* dir, const T* coeffs, const T* v_colors, T* v_dir) {
  v_dir[0] = v_dir[1] = v_dir[2] = 0;
  if (degree < 1) return;
  const T norm = std::sqrt(dir[0] * dir[0] + dir[1] * dir[1] + dir[2] * dir[2]);
  if (norm == T(0)) return;
  const T inorm = T(1) / norm;
  const T x = dir[0] * inorm, y = dir[1] * inorm, z = dir[2] * inorm;
  T dx[25] = {}, dy[25] = {}, dz[25] = {};
  const T C1 = T(0.48860251190292);
  dx[3] = -C1;
  dy[1] = -C1;
  dz[2] = C1;
  const T z2 = z * z;
  const T f_tmp0_b = T(-1.092548430592079) * z;
  const T f_c1 = x * x - y * y;
  const T f_s1 = T(2) * x * y;
  const T f_tmp0_b_z = T(-1.092548430592079);
  const T f_c1_x = T(2) * x, f_c1_y = T(-2) * y;
  const T f_s1_x = T(2) * y, f_s1_y = T(2) * x;
  const T p_sh6_z = T(2) * T(0.9461746957575601) * z;
  if (degree >= 2) {
    dx[4] = T(0.5462742152960395) * f_s1_x;
    dy[4] = T(0.5462742152960395) * f_s1_y;
    dy[5] = f_tmp0_b;
    dz[5] = f_tmp0_b_z * y;
    dz[6] = p_sh6_z;
    dx[7] = f_tmp0_b;
    dz[7] = f_tmp0_b_z * x;
    dx[8] = T(0.5462742152960395) * f_c1_x;
    dy[8] = T(0.5462742152960395) * f_c1_y;
  }
  const T f_tmp0_c = T(-2.285228997322329) * z2 + T(0.4570457994644658);
  const T f_tmp1_b = T(1.445305721320277) * z;
  const T f_c2 = x * f_c1 - y * f_s1;
  const T f_s2 = x * f_s1 + y * f_c1;
  const T p_sh12 = z * (T(1.865881662950577) * z2 - T(1.119528997770346));
  const T f_tmp0_c_z = T(-2.285228997322329) * T(2) * z;
  const T f_tmp1_b_z = T(1.445305721320277);
  const T f_c2_x = f_c1 + x * f_c1_x - y * f_s1_x;
  const T f_c2_y = x * f_c1_y - f_s1 - y * f_s1_y;
  const T f_s2_x = f_s1 + x * f_s1_x + y * f_c1_x;
  const T f_s2_y = x * f_s1_y + f_c1 + y * f_c1_y;
  const T p_sh12_z = T(3) * T(1.865881662950577) * z2 - T(1.119528997770346);
  if (degree >= 3) {
    dx[9] = T(-0.5900435899266435) * f_s2_x;
    dy[9] = T(-0.5900435899266435) * f_s2_y;
    dx[10] = f_tmp1_b * f_s1_x;
    dy[10] = f_tmp1_b * f_s1_y;
    dz[10] = f_tmp1_b_z * f_s1;
    dy[11] = f_tmp0_c;
    dz[11] = f_tmp0_c_z * y;
    dz[12] = p_sh12_z;
    dx[13] = f_tmp0_c;
    dz[13] = f_tmp0_c_z * x;
    dx[14] = f_tmp1_b * f_c1_x;
    dy[14] = f_tmp1_b * f_c1_y;
    dz[14] = f_tmp1_b_z * f_c1;
    dx[15] = T(-0.5900435899266435) * f_c2_x;
    dy[15] = T(-0.5900435899266435) * f_c2_y;
  }
  if (degree >= 4) {
    const T f_tmp0_d = z * (T(-4.683325804901025) * z2 + T(2.007139630671868));
    const T f_tmp1_c = T(3.31161143515146) * z2 - T(0.47308734787878);
    const T f_tmp2_b = T(-1.770130769779931) * z;
    const T f_tmp0_d_z = T(3) * T(-4.683325804901025) * z2 + T(2.007139630671868);
    const T f_tmp1_c_z = T(2) * T(3.31161143515146) * z;
    const T f_tmp2_b_z = T(-1.770130769779931);
    const T f_c3_x = f_c2 + x * f_c2_x - y * f_s2_x;
    const T f_c3_y = x * f_c2_y - f_s2 - y * f_s2_y;
    const T f_s3_x = f_s2 + y * f_c2_x + x * f_s2_x;
    const T f_s3_y = x * f_s2_y + f_c2 + y * f_c2_y;
    dx[16] = T(0.6258357354491763) * f_s3_x;
    dy[16] = T(0.6258357354491763) * f_s3_y;
    dx[17] = f_tmp2_b * f_s2_x;
    dy[17] = f_tmp2_b * f_s2_y;
    dz[17] = f_tmp2_b_z * f_s2;
    dx[18] = f_tmp1_c * f_s1_x;
    dy[18] = f_tmp1_c * f_s1_y;
    dz[18] = f_tmp1_c_z * f_s1;
    dy[19] = f_tmp0_d;
    dz[19] = f_tmp0_d_z * y;
    dz[20] = T(1.984313483298443) * (p_sh12 + z * p_sh12_z) - T(1.006230589874905) * p_sh6_z;
    dx[21] = f_tmp0_d;
    dz[21] = f_tmp0_d_z * x;
    dx[22] = f_tmp1_c * f_c1_x;
    dy[22] = f_tmp1_c * f_c1_y;
    dz[22] = f_tmp1_c_z * f_c1;
    dx[23] = f_tmp2_b * f_c2_x;
    dy[23] = f_tmp2_b * f_c2_y;
    dz[23] = f_tmp2_b_z * f_c2;
    dx[24] = T(0.6258357354491763) * f_c3_x;
    dy[24] = T(0.6258357354491763) * f_c3_y;
  }
  const int active = (degree + 1) * (degree + 1);
  T vn[3] = {0, 0, 0};
  for (int b = 1; b < active; ++b) {
    const T vb = coeffs[b * 3] * v_colors[0] + coeffs[b * 3 + 1] * v_colors[1] + coeffs[b * 3 + 2] * v_colors[2];
    vn[0] += dx[b] * vb;
    vn[1] += dy[b] * vb;
    vn[2] += dz[b] * vb;
  }
  const T dot = vn[0] * x + vn[1] * y + vn[2] * z;
  v_dir[0] = (vn[0] - dot * x) * inorm;
  v_dir[1] = (vn[1] - dot * y) * inorm;
  v_dir[2] = (vn[2] - dot * z) * inorm;
}

// GSPlatSphericalHarmonicsBackward::eval_cpu, gsplat_spherical_harmonics.cpp:503-554.
template <typename T>
void sh_backward(int degree, const T* dirs, const T* coeffs, const uint8_t* masks,
                 const T* v_colors, int64_t n, int64_t K, T* v_dirs, T* v_coeffs) {
  std::memset(v_coeffs, 0, sizeof(T) * n * K * 3);
  if (v_dirs) std::memset(v_dirs, 0, sizeof(T) * n * 3);
  const int active = (degree + 1) * (degree + 1);
  ORACLE_PARALLEL_FOR
  for (int64_t e = 0; e < n; ++e) {
    T basis[25];
    if (masks && !masks[e]) continue;
    sh_basis(degree, dirs + e * 3, basis);
    const T* vc = v_colors + e * 3;
    T* vco = v_coeffs + e * K * 3;
    for (int b = 0; b < active; ++b)
      for (int ch = 0; ch < 3; ++ch) vco[b * 3 + ch] = basis[b] * vc[ch];
    if (v_dirs) sh_dir_vjp(degree, dirs + e * 3, coeffs + e * K * 3, vc, v_dirs + e * 3);
  }
}

// ---------------------------------------------------------------------------
// Tile intersection, gsplat_intersect.cpp:60-112, 309-339, 433-485, 605-641.

int floor_log2_plus_one(int value) {
  return static_cast<int>(std::floor(std::log2(static_cast<float>(value)))) + 1;
}

struct Rect {
  int min_x, min_y, max_x, max_y;
};

Rect aabb_tile_rect(float mx, float my, int rx, int ry, int ts, int tw, int th) {
  if (rx <= 0 || ry <= 0) return {0, 0, 0, 0};
  const float trx = static_cast<float>(rx) / static_cast<float>(ts);
  const float try_ = static_cast<float>(ry) / static_cast<float>(ts);
  const float tx = mx / static_cast<float>(ts);
  const float ty = my / static_cast<float>(ts);
  Rect r;
  r.min_x = std::min(std::max(0, static_cast<int>(std::floor(tx - trx))), tw);
  r.min_y = std::min(std::max(0, static_cast<int>(std::floor(ty - try_))), th);
  r.max_x = std::min(std::max(0, static_cast<int>(std::ceil(tx + trx))), tw);
  r.max_y = std::min(std::max(0, static_cast<int>(std::ceil(ty + try_))), th);
  return r;
}

int64_t encode_isect_id(int image_id, int tile_id, float depth, int tile_n_bits) {
  uint32_t bits;
  std::memcpy(&bits, &depth, 4);
  return (static_cast<int64_t>(image_id) << (32 + tile_n_bits)) |
         (static_cast<int64_t>(tile_id) << 32) | static_cast<int64_t>(bits);
}

// ---------------------------------------------------------------------------
// Rasterization, gsplat_rasterize.cpp:249-369 (forward), 371-569 (backward).

// tile_evals (optional, [I, tile_height, tile_width]): per tile, the loop
// iterations of its pixels -- each entry evaluated before a pixel's
// termination, the terminating entry included (E_f).
template <typename T>
void raster_forward(const T* means2d, const T* conics, const T* colors, const T* opacities,
                    const T* backgrounds, const uint8_t* masks, const int32_t* tile_offsets,
                    const int32_t* flatten_ids, int64_t I, int64_t channels, int W, int H,
                    int tile_size, int tile_width, int tile_height, int64_t n_isects,
                    T* render_colors, T* render_alphas, int32_t* last_ids, int64_t* tile_evals = nullptr) {
  std::memset(render_colors, 0, sizeof(T) * I * H * W * channels);
  ORACLE_PARALLEL_TILES
  for (int64_t image = 0; image < I; ++image)
    for (int ty = 0; ty < tile_height; ++ty)
      for (int tx = 0; tx < tile_width; ++tx) {
        const int tile = ty * tile_width + tx;
        const int64_t oi = image * tile_height * tile_width + tile;
        const int64_t start = tile_offsets[oi];
        const int64_t end = (image == I - 1 && tile == tile_width * tile_height - 1) ? n_isects : tile_offsets[oi + 1];
        const bool skip = masks && !masks[oi];
        int64_t evals = 0;
        for (int ly = 0; ly < tile_size; ++ly) {
          const int y = ty * tile_size + ly;
          if (y >= H) continue;
          for (int lx = 0; lx < tile_size; ++lx) {
            const int x = tx * tile_size + lx;
            if (x >= W) continue;
            const int64_t pix = image * H * W + static_cast<int64_t>(y) * W + x;
            const T px = T(x) + T(0.5), py = T(y) + T(0.5);
            T Tr = 1;
            int32_t cur = 0;
            T* out = render_colors + pix * channels;
            for (int64_t idx = start; !skip && idx < end; ++idx) {
              ++evals;
              const int64_t g = flatten_ids[idx];
              const T dx = means2d[g * 2] - px;
              const T dy = means2d[g * 2 + 1] - py;
              const T c0 = conics[g * 3], c1 = conics[g * 3 + 1], c2 = conics[g * 3 + 2];
              const T sigma = T(0.5) * (c0 * dx * dx + c2 * dy * dy) + c1 * dx * dy;
              const T alpha = std::min(T(kMaxAlpha), opacities[g] * std::exp(-sigma));
              if (sigma < T(0) || alpha < T(kAlphaThreshold)) continue;
              const T next_T = Tr * (T(1) - alpha);
              if (next_T <= T(kTransmittanceThreshold)) break;
              const T vis = alpha * Tr;
              for (int64_t ch = 0; ch < channels; ++ch) out[ch] += colors[g * channels + ch] * vis;
              cur = static_cast<int32_t>(idx);
              Tr = next_T;
            }
            render_alphas[pix] = T(1) - Tr;
            for (int64_t ch = 0; ch < channels; ++ch)
              out[ch] += Tr * (backgrounds ? backgrounds[image * channels + ch] : T(0));
            last_ids[pix] = cur;
          }
        }
        if (tile_evals) tile_evals[oi] = evals;
      }
}

template <typename T>
void raster_backward(const T* means2d, const T* conics, const T* colors, const T* opacities,
                     const T* backgrounds, const uint8_t* masks, const int32_t* tile_offsets,
                     const int32_t* flatten_ids, int64_t I, int64_t N, int64_t channels, int W,
                     int H, int tile_size, int tile_width, int tile_height, int64_t n_isects,
                     const T* render_alphas, const int32_t* last_ids, const T* v_render_colors,
                     const T* v_render_alphas, T* v_means2d_abs, T* v_means2d, T* v_conics,
                     T* v_colors, T* v_opacities, T* v_backgrounds) {
  const int64_t G = I * N;
  if (v_means2d_abs) std::memset(v_means2d_abs, 0, sizeof(T) * G * 2);
  std::memset(v_means2d, 0, sizeof(T) * G * 2);
  std::memset(v_conics, 0, sizeof(T) * G * 3);
  std::memset(v_colors, 0, sizeof(T) * G * channels);
  std::memset(v_opacities, 0, sizeof(T) * G);
  if (v_backgrounds) std::memset(v_backgrounds, 0, sizeof(T) * I * channels);
  // gradient sums are shared across tiles: atomic adds when the tiles run on
  // several threads
  ORACLE_PARALLEL_TILES
  for (int64_t image = 0; image < I; ++image)
    for (int ty = 0; ty < tile_height; ++ty)
      for (int tx = 0; tx < tile_width; ++tx) {
        std::vector<int64_t> ids;
        std::vector<T> alphas, viss, buffer(channels);
        const int tile = ty * tile_width + tx;
        const int64_t oi = image * tile_height * tile_width + tile;
        if (masks && !masks[oi]) continue;
        const int64_t start = tile_offsets[oi];
        const int64_t end = (image == I - 1 && tile == tile_width * tile_height - 1) ? n_isects : tile_offsets[oi + 1];
        for (int ly = 0; ly < tile_size; ++ly) {
          const int y = ty * tile_size + ly;
          if (y >= H) continue;
          for (int lx = 0; lx < tile_size; ++lx) {
            const int x = tx * tile_size + lx;
            if (x >= W) continue;
            const int64_t pix = image * H * W + static_cast<int64_t>(y) * W + x;
            const int64_t bin_final = last_ids[pix];
            ids.clear();
            alphas.clear();
            viss.clear();
            const T px = T(x) + T(0.5), py = T(y) + T(0.5);
            for (int64_t idx = start; idx < end && idx <= bin_final; ++idx) {
              const int64_t g = flatten_ids[idx];
              const T dx = means2d[g * 2] - px;
              const T dy = means2d[g * 2 + 1] - py;
              const T c0 = conics[g * 3], c1 = conics[g * 3 + 1], c2 = conics[g * 3 + 2];
              const T sigma = T(0.5) * (c0 * dx * dx + c2 * dy * dy) + c1 * dx * dy;
              const T vis = std::exp(-sigma);
              const T alpha = std::min(T(kMaxAlpha), opacities[g] * vis);
              if (sigma < T(0) || alpha < T(kAlphaThreshold)) continue;
              ids.push_back(idx);
              alphas.push_back(alpha);
              viss.push_back(vis);
            }
            const T T_final = T(1) - render_alphas[pix];
            T Tr = T_final;
            std::fill(buffer.begin(), buffer.end(), T(0));
            const T v_ra = v_render_alphas[pix];
            const T* v_rc = v_render_colors + pix * channels;
            if (v_backgrounds)
              for (int64_t ch = 0; ch < channels; ++ch) {
                ORACLE_ATOMIC
                v_backgrounds[image * channels + ch] += T_final * v_rc[ch];
              }
            for (int64_t l = static_cast<int64_t>(ids.size()) - 1; l >= 0; --l) {
              const int64_t g = flatten_ids[ids[l]];
              const T alpha = alphas[l], vis = viss[l];
              const T ra = T(1) / std::max(T(kMinOneMinusAlpha), T(1) - alpha);
              Tr *= ra;
              const T fac = alpha * Tr;
              for (int64_t ch = 0; ch < channels; ++ch) {
                ORACLE_ATOMIC
                v_colors[g * channels + ch] += fac * v_rc[ch];
              }
              T v_alpha = 0;
              for (int64_t ch = 0; ch < channels; ++ch)
                v_alpha += (colors[g * channels + ch] * Tr - buffer[ch] * ra) * v_rc[ch];
              v_alpha += T_final * ra * v_ra;
              if (backgrounds) {
                T accum = 0;
                for (int64_t ch = 0; ch < channels; ++ch) accum += backgrounds[image * channels + ch] * v_rc[ch];
                v_alpha += -T_final * ra * accum;
              }
              if (opacities[g] * vis <= T(kMaxAlpha)) {
                const T dx = means2d[g * 2] - px;
                const T dy = means2d[g * 2 + 1] - py;
                const T c0 = conics[g * 3], c1 = conics[g * 3 + 1], c2 = conics[g * 3 + 2];
                const T v_sigma = -opacities[g] * vis * v_alpha;
                const T v_x = v_sigma * (c0 * dx + c1 * dy);
                const T v_y = v_sigma * (c1 * dx + c2 * dy);
                const T vc0 = T(0.5) * v_sigma * dx * dx, vc1 = v_sigma * dx * dy;
                const T vc2 = T(0.5) * v_sigma * dy * dy, vo = vis * v_alpha;
                ORACLE_ATOMIC
                v_conics[g * 3] += vc0;
                ORACLE_ATOMIC
                v_conics[g * 3 + 1] += vc1;
                ORACLE_ATOMIC
                v_conics[g * 3 + 2] += vc2;
                ORACLE_ATOMIC
                v_means2d[g * 2] += v_x;
                ORACLE_ATOMIC
                v_means2d[g * 2 + 1] += v_y;
                if (v_means2d_abs) {
                  const T ax = std::fabs(v_x), ay = std::fabs(v_y);
                  ORACLE_ATOMIC
                  v_means2d_abs[g * 2] += ax;
                  ORACLE_ATOMIC
                  v_means2d_abs[g * 2 + 1] += ay;
                }
                ORACLE_ATOMIC
                v_opacities[g] += vo;
              }
              for (int64_t ch = 0; ch < channels; ++ch) buffer[ch] += colors[g * channels + ch] * fac;
            }
          }
        }
      }
}

}  // namespace

// ---------------------------------------------------------------------------
// extern "C" surface for ctypes. Suffix _f32 / _f64 selects the scalar type.

#define ORACLE_INSTANTIATE(T, SFX)                                                               \
  extern "C" void oracle_quat_scale_to_covar_preci_fwd_##SFX(                                    \
      const T* quats, const T* scales, int64_t n, int compute_covar, int compute_preci, int triu, \
      T* covars, T* precis) {                                                                    \
    qs_forward<T>(quats, scales, n, compute_covar, compute_preci, triu, covars, precis);         \
  }                                                                                              \
  extern "C" void oracle_quat_scale_to_covar_preci_bwd_##SFX(                                    \
      const T* quats, const T* scales, const T* v_covars, const T* v_precis, int64_t n, int triu, \
      T* v_quats, T* v_scales) {                                                                 \
    qs_backward<T>(quats, scales, v_covars, v_precis, n, triu, v_quats, v_scales);               \
  }                                                                                              \
  extern "C" void oracle_projection_fwd_##SFX(                                                   \
      const T* means, const T* covars, const T* quats, const T* scales, const T* opacities,       \
      const T* viewmats, const T* Ks, int64_t B, int64_t C, int64_t N, const ProjParams* p,      \
      int32_t* radii, T* means2d, T* depths, T* conics, T* compensations) {                      \
    proj_forward<T>(means, covars, quats, scales, opacities, viewmats, Ks, B, C, N, *p, radii,   \
                    means2d, depths, conics, compensations);                                     \
  }                                                                                              \
  extern "C" void oracle_projection_bwd_##SFX(                                                   \
      const T* means, const T* covars, const T* quats, const T* scales, const T* viewmats,        \
      const T* Ks, int64_t B, int64_t C, int64_t N, const ProjParams* p, const int32_t* radii,   \
      const T* conics, const T* compensations, const T* v_means2d, const T* v_depths,            \
      const T* v_conics, const T* v_compensations, T* v_means, T* v_covars, T* v_quats,          \
      T* v_scales, T* v_viewmats) {                                                              \
    proj_backward<T>(means, covars, quats, scales, viewmats, Ks, B, C, N, *p, radii, conics,     \
                     compensations, v_means2d, v_depths, v_conics, v_compensations, v_means,     \
                     v_covars, v_quats, v_scales, v_viewmats);                                   \
  }                                                                                              \
  extern "C" void oracle_sh_fwd_##SFX(int degree, const T* dirs, const T* coeffs,                 \
                                      const uint8_t* masks, int64_t n, int64_t K, T* colors) {   \
    sh_forward<T>(degree, dirs, coeffs, masks, n, K, colors);                                    \
  }                                                                                              \
  extern "C" void oracle_sh_bwd_##SFX(int degree, const T* dirs, const T* coeffs,                 \
                                      const uint8_t* masks, const T* v_colors, int64_t n,        \
                                      int64_t K, T* v_dirs, T* v_coeffs) {                       \
    sh_backward<T>(degree, dirs, coeffs, masks, v_colors, n, K, v_dirs, v_coeffs);               \
  }                                                                                              \
  extern "C" void oracle_raster_fwd_##SFX(                                                       \
      const T* means2d, const T* conics, const T* colors, const T* opacities,                   \
      const T* backgrounds, const uint8_t* masks, const int32_t* tile_offsets,                   \
      const int32_t* flatten_ids, int64_t I, int64_t channels, int W, int H, int tile_size,      \
      int tile_width, int tile_height, int64_t n_isects, T* render_colors, T* render_alphas,     \
      int32_t* last_ids, int64_t* tile_evals) {                                                  \
    raster_forward<T>(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets,      \
                      flatten_ids, I, channels, W, H, tile_size, tile_width, tile_height,        \
                      n_isects, render_colors, render_alphas, last_ids, tile_evals);             \
  }                                                                                              \
  extern "C" void oracle_raster_bwd_##SFX(                                                       \
      const T* means2d, const T* conics, const T* colors, const T* opacities,                   \
      const T* backgrounds, const uint8_t* masks, const int32_t* tile_offsets,                   \
      const int32_t* flatten_ids, int64_t I, int64_t N, int64_t channels, int W, int H,          \
      int tile_size, int tile_width, int tile_height, int64_t n_isects, const T* render_alphas,  \
      const int32_t* last_ids, const T* v_render_colors, const T* v_render_alphas,               \
      T* v_means2d_abs, T* v_means2d, T* v_conics, T* v_colors, T* v_opacities,                  \
      T* v_backgrounds) {                                                                        \
    raster_backward<T>(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets,     \
                       flatten_ids, I, N, channels, W, H, tile_size, tile_width, tile_height,    \
                       n_isects, render_alphas, last_ids, v_render_colors, v_render_alphas,      \
                       v_means2d_abs, v_means2d, v_conics, v_colors, v_opacities,                \
                       v_backgrounds);                                                           \
  }

ORACLE_INSTANTIATE(float, f32)
ORACLE_INSTANTIATE(double, f64)

extern "C" {

int oracle_floor_log2_plus_one(int value) { return floor_log2_plus_one(value); }

// GSPlatIntersectTileCount::eval_cpu, gsplat_intersect.cpp:309-339.
void oracle_isect_count(const float* means2d, const int32_t* radii, int64_t numel, int tile_size,
                        int tile_width, int tile_height, int32_t* tiles_per_gauss) {
  ORACLE_PARALLEL_FOR
  for (int64_t i = 0; i < numel; ++i) {
    const Rect r = aabb_tile_rect(means2d[i * 2], means2d[i * 2 + 1], radii[i * 2], radii[i * 2 + 1],
                                  tile_size, tile_width, tile_height);
    tiles_per_gauss[i] = (r.max_y - r.min_y) * (r.max_x - r.min_x);
  }
}

// Exclusive scan replacing mx::cumsum(inclusive=false), gsplat_intersect.cpp:196-211.
// Returns the total (offsets[last] + counts[last], gsplat_intersect.cpp:155-170).
int64_t oracle_exclusive_scan(const int32_t* counts, int64_t n, int32_t* offsets) {
  int64_t acc = 0;
  for (int64_t i = 0; i < n; ++i) {
    offsets[i] = static_cast<int32_t>(acc);
    acc += counts[i];
  }
  return acc;
}

// GSPlatIntersectTileEncode::eval_cpu, gsplat_intersect.cpp:433-485.
int oracle_isect_encode(const float* means2d, const int32_t* radii, const float* depths,
                        const int32_t* offsets, int64_t I, int64_t numel, int tile_size,
                        int tile_width, int tile_height, int64_t total, int64_t* isect_ids,
                        int32_t* flatten_ids) {
  const int64_t n_per_image = numel / I;
  const int tile_n_bits = floor_log2_plus_one(tile_width * tile_height);
  int bad = 0;  // an offset outside [0, total): inconsistent inputs
  ORACLE_PARALLEL_FOR
  for (int64_t idx = 0; idx < numel; ++idx) {
    const int image_id = static_cast<int>(idx / n_per_image);
    const Rect r = aabb_tile_rect(means2d[idx * 2], means2d[idx * 2 + 1], radii[idx * 2],
                                  radii[idx * 2 + 1], tile_size, tile_width, tile_height);
    int64_t o = offsets[idx];
    for (int ty = r.min_y; ty < r.max_y; ++ty)
      for (int tx = r.min_x; tx < r.max_x; ++tx) {
        if (o < 0 || o >= total) {
          ORACLE_ATOMIC
          bad |= 1;
          ty = r.max_y;
          break;
        }
        isect_ids[o] = encode_isect_id(image_id, ty * tile_width + tx, depths[idx], tile_n_bits);
        flatten_ids[o] = static_cast<int32_t>(idx);
        ++o;
      }
  }
  return bad ? -1 : 0;
}

// Ellipse ("AccuTile") tiles: the use_conics / use_opacities path that the
// reference rejects (gsplat_intersect.cpp:123-126) and that lives in upstream
// gsplat's IntersectTile.cu, a dependency absent from the reference tree
// (Task_Metal.md:95-115, note/gsplat_cuda_source_map.md:359-360). Restated
// from the published method (Speedy-Splat, Hanson et al., CVPR 2025: SnugBox
// bounds from the opacity-aware threshold, AccuTile exact tile rows) with the
// rasterizer's threshold alpha >= 1/255 and its cull slack: the ellipse
// d^T Q d <= 2 (1.05 ln(255 o) + 1e-4), intersected with the AABB rect, tile
// row by tile row over the row's pixel-centre slab. Rows are listed
// row-major, so encode keeps the reference's per-Gaussian order.
// Parity: pinned against brute force in tests/test_oracle_isect.py (every
// pixel that passes the rasterizer's float32 alpha test lies in a listed
// tile; every listed tile meets the slack ellipse, every tile that meets it
// with margin is listed, by a rectangle-minimum formulation in float64) and
// by rendering identity (AccuTile lists render the same image as AABB lists).
// Upstream's own tile ids are unpinned here (no fixture of them exists).

// ln z, z finite > 0, by frexp and the atanh series (same float operations
// as the device code, so both give the same bits).
float ellipse_log(float z) {
  int e = 0;
  float m = std::frexp(z, &e);
  if (m < 0.70710678f) {
    m = m * 2.0f;
    e = e - 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 0.11111111f;
  p = p * s2 + 0.14285715f;
  p = p * s2 + 0.2f;
  p = p * s2 + 0.33333334f;
  p = p * s2 + 1.0f;
  return static_cast<float>(e) * 0.69314718f + 2.0f * s * p;
}

// Column ranges [c0, c1) of the Gaussian's tiles, one per row of its rect.
struct EllipseRows {
  Rect r;
  std::vector<int> c0, c1;  // indexed by ty - r.min_y
};

EllipseRows ellipse_rows(const float* means2d, const int32_t* radii, const float* conics,
                         const float* opacities, int64_t g, int ts, int tw, int th) {
  const float mx = means2d[g * 2], my = means2d[g * 2 + 1];
  EllipseRows out;
  out.r = aabb_tile_rect(mx, my, radii[g * 2], radii[g * 2 + 1], ts, tw, th);
  const Rect& r = out.r;
  if (r.max_x <= r.min_x || r.max_y <= r.min_y) return out;
  const int rows = r.max_y - r.min_y;
  const float o = opacities[g];
  if (o <= 0.0f) {  // alpha <= 0 everywhere
    out.c0.assign(rows, r.min_x);
    out.c1.assign(rows, r.min_x);
    return out;
  }
  // whole rect where the threshold or the conic is unusable
  out.c0.assign(rows, r.min_x);
  out.c1.assign(rows, r.max_x);
  const float a = conics[g * 3], b = conics[g * 3 + 1], c = conics[g * 3 + 2];
  const float z = 255.0f * o;
  if (!(z < 3.0e38f) || !(a > 0.0f && c > 0.0f && a < 1.0e30f && c < 1.0e30f) || !(std::fabs(mx) < 1.0e30f) ||
      !(std::fabs(my) < 1.0e30f))
    return out;
  const float det = a * c - b * b;
  if (!(det > 1.0e-4f * a * c)) return out;
  const float lim = 1.05f * ellipse_log(z) + 1.0e-4f;
  if (!(lim >= 0.0f)) {
    out.c1 = out.c0;
    return out;
  }
  const float R = 2.0f * lim;
  const float x_ext = std::sqrt(R * c / det);
  const float y_ext = std::sqrt(R * a / det);
  const float aR = a * R;
  const float dy_left = b * x_ext / c;  // leftmost point's dy; rightmost at -dy_left
  const float fts = static_cast<float>(ts);
  for (int ty = r.min_y; ty < r.max_y; ++ty) {
    int& lo_col = out.c0[ty - r.min_y];
    int& hi_col = out.c1[ty - r.min_y];
    const float top = static_cast<float>(ty * ts) + 0.5f;  // first pixel centre of the row
    const float bottom = top + static_cast<float>(ts - 1);
    const float d0 = std::fmax(top - my, -y_ext);
    const float d1 = std::fmin(bottom - my, y_ext);
    if (!(d0 <= d1)) {
      hi_col = lo_col = r.min_x;
      continue;
    }
    const float dl = std::fmin(std::fmax(dy_left, d0), d1);
    const float dr = std::fmin(std::fmax(-dy_left, d0), d1);
    const float half_l = std::sqrt(std::fmax(aR - det * dl * dl, 0.0f));
    const float half_r = std::sqrt(std::fmax(aR - det * dr * dr, 0.0f));
    const float xl = mx - (b * dl + half_l) / a;
    const float xr = mx + (half_r - b * dr) / a;
    // columns whose pixel centres tx ts + 1/2 .. tx ts + ts - 1/2 meet [xl, xr]
    const float first = std::floor((xl + 0.5f) / fts);
    const float end = std::floor((xr - 0.5f) / fts) + 1.0f;
    const float fmin = static_cast<float>(r.min_x), fmax = static_cast<float>(r.max_x);
    lo_col = static_cast<int>(std::fmin(std::fmax(first, fmin), fmax));
    hi_col = static_cast<int>(std::fmin(std::fmax(end, fmin), fmax));
  }
  return out;
}

// argsort + take, gsplat_intersect.cpp:266-286, as a stable sort.
void oracle_isect_sort(const int64_t* keys, const int32_t* vals, int64_t m, int64_t* keys_out,
                       int32_t* vals_out) {
  std::vector<int64_t> order(m);
  std::iota(order.begin(), order.end(), 0);
#ifdef _OPENMP
  __gnu_parallel::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return keys[a] < keys[b]; });
#else
  std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return keys[a] < keys[b]; });
#endif
  for (int64_t i = 0; i < m; ++i) {
    keys_out[i] = keys[order[i]];
    vals_out[i] = vals[order[i]];
  }
}

// Ellipse tile counts (the AccuTile count: sum of the row widths).
void oracle_isect_count_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                 const float* opacities, int64_t numel, int tile_size, int tile_width,
                                 int tile_height, int32_t* tiles_per_gauss) {
  for (int64_t i = 0; i < numel; ++i) {
    const EllipseRows e = ellipse_rows(means2d, radii, conics, opacities, i, tile_size, tile_width, tile_height);
    int32_t n = 0;
    for (size_t k = 0; k < e.c0.size(); ++k) n += std::max(e.c1[k] - e.c0[k], 0);
    tiles_per_gauss[i] = n;
  }
}

// Ellipse tile encode: pair-major, row-major within each pair, ids as the
// AABB encode's.
int oracle_isect_encode_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                 const float* opacities, const float* depths, const int32_t* offsets, int64_t I,
                                 int64_t numel, int tile_size, int tile_width, int tile_height, int64_t total,
                                 int64_t* isect_ids, int32_t* flatten_ids) {
  const int64_t n_per_image = numel / I;
  const int tile_n_bits = floor_log2_plus_one(tile_width * tile_height);
  for (int64_t idx = 0; idx < numel; ++idx) {
    const int image_id = static_cast<int>(idx / n_per_image);
    const EllipseRows e = ellipse_rows(means2d, radii, conics, opacities, idx, tile_size, tile_width, tile_height);
    int64_t o = offsets[idx];
    for (size_t k = 0; k < e.c0.size(); ++k) {
      const int ty = e.r.min_y + static_cast<int>(k);
      for (int tx = e.c0[k]; tx < e.c1[k]; ++tx) {
        if (o < 0 || o >= total) return -1;
        isect_ids[o] = encode_isect_id(image_id, ty * tile_width + tx, depths[idx], tile_n_bits);
        flatten_ids[o] = static_cast<int32_t>(idx);
        ++o;
      }
    }
  }
  return 0;
}

// Packed-layout encode (IntersectTileParams.packed, which the reference
// rejects at gsplat_intersect.cpp:115-118; upstream gsplat's isect_tiles with
// image_ids): row idx of nnz belongs to image image_ids[idx] and its flatten
// id is idx; tiles are the AABB rect's, or the ellipse rows when conics and
// opacities are given. Otherwise the dense encode order.
int oracle_isect_encode_packed(const float* means2d, const int32_t* radii, const float* conics,
                               const float* opacities, const int32_t* image_ids, const float* depths,
                               const int32_t* offsets, int64_t nnz, int tile_size, int tile_width, int tile_height,
                               int64_t total, int64_t* isect_ids, int32_t* flatten_ids) {
  const int tile_n_bits = floor_log2_plus_one(tile_width * tile_height);
  for (int64_t idx = 0; idx < nnz; ++idx) {
    EllipseRows e;
    if (conics && opacities) {
      e = ellipse_rows(means2d, radii, conics, opacities, idx, tile_size, tile_width, tile_height);
    } else {
      e.r = aabb_tile_rect(means2d[idx * 2], means2d[idx * 2 + 1], radii[idx * 2], radii[idx * 2 + 1], tile_size,
                           tile_width, tile_height);
      const int rows = std::max(e.r.max_y - e.r.min_y, 0);
      e.c0.assign(rows, e.r.min_x);
      e.c1.assign(rows, e.r.max_x);
    }
    int64_t o = offsets[idx];
    for (size_t k = 0; k < e.c0.size(); ++k) {
      const int ty = e.r.min_y + static_cast<int>(k);
      for (int tx = e.c0[k]; tx < e.c1[k]; ++tx) {
        if (o < 0 || o >= total) return -1;
        isect_ids[o] = encode_isect_id(image_ids[idx], ty * tile_width + tx, depths[idx], tile_n_bits);
        flatten_ids[o] = static_cast<int32_t>(idx);
        ++o;
      }
    }
  }
  return 0;
}

// rasterize_to_indices (upstream gsplat's rasterize_to_indices_in_range,
// note/gsplat_cuda_source_map.md:494-545; not in the reference): per pixel,
// from transmittances[pix] (NULL: 1), the entries at list positions
// [range_start, range_end) of its tile that the float32 forward loop above
// composites (same alpha, threshold and stopping rule), in list order.
// counts (pass 1) or, with starts, gauss_ids / indices (pass 2).
void oracle_raster_indices(int64_t range_start, int64_t range_end, const float* transmittances,
                           const float* means2d, const float* conics, const float* opacities,
                           const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I, int W, int H,
                           int tile_size, int tile_width, int tile_height, int64_t n_isects, int32_t* counts,
                           const int32_t* starts, int32_t* gauss_ids, int64_t* indices) {
  const int64_t n_tiles = static_cast<int64_t>(tile_width) * tile_height;
  for (int64_t image = 0; image < I; ++image)
    for (int y = 0; y < H; ++y)
      for (int x = 0; x < W; ++x) {
        const int64_t tile = (y / tile_size) * tile_width + (x / tile_size);
        const int64_t oi = image * n_tiles + tile;
        const int64_t t0 = tile_offsets[oi];
        const int64_t t1 = (oi + 1 == I * n_tiles) ? n_isects : tile_offsets[oi + 1];
        const int64_t start = std::min(t0 + range_start, t1), end = std::min(t0 + range_end, t1);
        const int64_t pix = (image * H + y) * W + x;
        const float px = static_cast<float>(x) + 0.5f, py = static_cast<float>(y) + 0.5f;
        float Tr = transmittances ? transmittances[pix] : 1.0f;
        int64_t pos = starts ? starts[pix] : 0;
        int32_t cnt = 0;
        for (int64_t idx = start; idx < end; ++idx) {
          const int64_t g = flatten_ids[idx];
          const float dx = means2d[g * 2] - px;
          const float dy = means2d[g * 2 + 1] - py;
          const float c0 = conics[g * 3], c1 = conics[g * 3 + 1], c2 = conics[g * 3 + 2];
          const float sigma = 0.5f * (c0 * dx * dx + c2 * dy * dy) + c1 * dx * dy;
          const float alpha = std::min(kMaxAlpha, opacities[g] * std::exp(-sigma));
          if (sigma < 0.0f || alpha < kAlphaThreshold) continue;
          const float next_T = Tr * (1.0f - alpha);
          if (next_T <= kTransmittanceThreshold) break;
          if (starts) {
            gauss_ids[pos] = static_cast<int32_t>(g);
            indices[pos] = pix;
            ++pos;
          }
          ++cnt;
          Tr = next_T;
        }
        if (counts) counts[pix] = cnt;
      }
}

// Threads of the OpenMP build's parallel loops (the CPU baseline times 1 and
// all); returns the count in effect, 1 for a build without OpenMP.
int oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}

// CPU baseline only (never for comparisons): flush denormal results and inputs
// to zero on the calling thread and every OpenMP thread, as a tuned CPU run
// would; tiny cotangents otherwise make x86 take its slow denormal path in
// whole stages. Returns 1 where the control exists (x86-64), else 0.
int oracle_flush_denormals(void) {
#if defined(__x86_64__)
  _mm_setcsr(_mm_getcsr() | 0x8040u);  // FTZ | DAZ
#ifdef _OPENMP
#pragma omp parallel
  _mm_setcsr(_mm_getcsr() | 0x8040u);
#endif
  return 1;
#else
  return 0;
#endif
}

// GSPlatIntersectOffset::eval_cpu, gsplat_intersect.cpp:605-641.
void oracle_isect_offset(const int64_t* isect_ids, int64_t n_isects, int I, int tile_width,
                         int tile_height, int32_t* offsets) {
  const int n_tiles = tile_width * tile_height;
  const int tile_n_bits = floor_log2_plus_one(n_tiles);
  const int64_t n_offsets = static_cast<int64_t>(I) * n_tiles;
  ORACLE_PARALLEL_FOR
  for (int64_t o = 0; o < n_offsets; ++o) {
    const int64_t key = ((o / n_tiles) << tile_n_bits) | (o % n_tiles);
    int64_t lo = 0, hi = n_isects;
    while (lo < hi) {
      const int64_t mid = lo + (hi - lo) / 2;
      if ((isect_ids[mid] >> 32) < key)
        lo = mid + 1;
      else
        hi = mid;
    }
    offsets[o] = static_cast<int32_t>(lo);
  }
}

}  // extern "C"
