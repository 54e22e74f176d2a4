// Real spherical harmonics (degrees 0..4), forward / backward, for gfx950.
//
// Layout is the reference's AoS: coeffs [n, K, 3], 12*K bytes per Gaussian.
// A block of kShBlock Gaussians stages the active (degree+1)^2 bases of its
// rows through LDS with consecutive lanes reading consecutive floats, so the
// HBM stream is read once, coalesced, instead of each lane striding 12*K
// bytes. The backward writes v_coeffs the same way: each lane computes its
// Gaussian's basis into LDS, then the block writes the [kShBlock, K, 3] slab
// with consecutive lanes on consecutive floats. Index splits use exact
// multiply-high reciprocals (valid for the block-slab index range).
//
// Math follows gsplat_core/gsplat_spherical_harmonics.cpp:112-425 in the same
// operation order (FMA contraction off for this file).
#include "common.hpp"
#include "packed_ranks.hpp"

namespace gsplat_hip {
namespace {

constexpr int kShBlock = 128;
constexpr float kC0 = 0.2820947917738781f;
constexpr float kC1 = 0.48860251190292f;

// floor(i / d) for i * (m*d - 2^32) < 2^32, with m = ceil(2^32 / d).
__host__ __device__ inline uint32_t magic_for(uint32_t d) {
  return static_cast<uint32_t>((0x100000000ull + d - 1) / d);
}
__device__ __forceinline__ uint32_t fast_div(uint32_t i, uint32_t m) { return __umulhi(i, m); }

// gsplat_spherical_harmonics.cpp:112-187
template <int DEG>
__device__ __forceinline__ void sh_basis(float dx, float dy, float dz, float* basis) {
  constexpr int A = (DEG + 1) * (DEG + 1);
#pragma unroll
  for (int i = 0; i < A; ++i) basis[i] = 0.0f;
  basis[0] = kC0;
  if (DEG < 1) return;
  const float norm = sqrtf(dx * dx + dy * dy + dz * dz);
  if (norm == 0.0f) return;
  const float x = dx / norm, y = dy / norm, z = dz / norm;
  basis[1] = -kC1 * y;
  basis[2] = kC1 * z;
  basis[3] = -kC1 * x;
  if (DEG < 2) return;
  const float z2 = z * z;
  const float f_tmp0_b = -1.092548430592079f * z;
  const float f_c1 = x * x - y * y;
  const float f_s1 = 2.0f * x * y;
  basis[4] = 0.5462742152960395f * f_s1;
  basis[5] = f_tmp0_b * y;
  basis[6] = 0.9461746957575601f * z2 - 0.3153915652525201f;
  basis[7] = f_tmp0_b * x;
  basis[8] = 0.5462742152960395f * f_c1;
  if (DEG < 3) return;
  const float f_tmp0_c = -2.285228997322329f * z2 + 0.4570457994644658f;
  const float f_tmp1_b = 1.445305721320277f * z;
  const float f_c2 = x * f_c1 - y * f_s1;
  const float f_s2 = x * f_s1 + y * f_c1;
  basis[9] = -0.5900435899266435f * f_s2;
  basis[10] = f_tmp1_b * f_s1;
  basis[11] = f_tmp0_c * y;
  basis[12] = z * (1.865881662950577f * z2 - 1.119528997770346f);
  basis[13] = f_tmp0_c * x;
  basis[14] = f_tmp1_b * f_c1;
  basis[15] = -0.5900435899266435f * f_c2;
  if (DEG < 4) return;
  const float f_tmp0_d = z * (-4.683325804901025f * z2 + 2.007139630671868f);
  const float f_tmp1_c = 3.31161143515146f * z2 - 0.47308734787878f;
  const float f_tmp2_b = -1.770130769779931f * z;
  const float f_c3 = x * f_c2 - y * f_s2;
  const float f_s3 = x * f_s2 + y * f_c2;
  basis[16] = 0.6258357354491763f * f_s3;
  basis[17] = f_tmp2_b * f_s2;
  basis[18] = f_tmp1_c * f_s1;
  basis[19] = f_tmp0_d * y;
  basis[20] = 1.984313483298443f * z * basis[12] - 1.006230589874905f * basis[6];
  basis[21] = f_tmp0_d * x;
  basis[22] = f_tmp1_c * f_c1;
  basis[23] = f_tmp2_b * f_c2;
  basis[24] = 0.6258357354491763f * f_c3;
}

// LDS row stride for W floats per row: odd, so lanes reading the same column
// of consecutive rows hit distinct banks.
__host__ __device__ constexpr int padded(int w) { return w | 1; }

// Copies the first W = A*3 floats of `cnt` rows (row stride k3 floats in
// global memory) into LDS rows of stride padded(W). The block's rows are one
// contiguous span of cnt*k3 floats; it is read front to back with 16-byte
// loads when aligned (unrolled for more loads in flight), else 4-byte loads.
template <int A>
__device__ __forceinline__ void stage_rows(float* __restrict__ lds, const float* __restrict__ src, int cnt,
                                           uint32_t k3, uint32_t k3_magic) {
  constexpr int W = A * 3;
  constexpr int PW = padded(W);
  const uint32_t total = static_cast<uint32_t>(cnt) * k3;
  auto put = [&](uint32_t f, float v) {
    const uint32_t r = fast_div(f, k3_magic);
    const uint32_t c = f - r * k3;
    if (c < static_cast<uint32_t>(W)) lds[r * PW + c] = v;
  };
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0 && (total & 3) == 0) {
    const float4* src4 = reinterpret_cast<const float4*>(src);
    const uint32_t total4 = total >> 2;
#pragma unroll 4
    for (uint32_t i = threadIdx.x; i < total4; i += kShBlock) {
      const float4 v = src4[i];
      put(4 * i, v.x);
      put(4 * i + 1, v.y);
      put(4 * i + 2, v.z);
      put(4 * i + 3, v.w);
    }
  } else {
#pragma unroll 4
    for (uint32_t i = threadIdx.x; i < total; i += kShBlock) put(i, src[i]);
  }
}

template <int DEG>
__global__ void __launch_bounds__(kShBlock) sh_fwd_kernel(const float* __restrict__ dirs,
                                                          const float* __restrict__ coeffs,
                                                          const uint8_t* __restrict__ masks, int64_t n, int64_t K,
                                                          uint32_t k3_magic, float* __restrict__ colors) {
  constexpr int A = (DEG + 1) * (DEG + 1);
  constexpr int PW = padded(A * 3);
  __shared__ float sc[kShBlock * PW];
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kShBlock;
  const int cnt = static_cast<int>(min<int64_t>(kShBlock, n - e0));
  stage_rows<A>(sc, coeffs + e0 * K * 3, cnt, static_cast<uint32_t>(K * 3), k3_magic);
  __syncthreads();
  const int t = threadIdx.x;
  if (t >= cnt) return;
  const int64_t e = e0 + t;
  float out[3] = {0.0f, 0.0f, 0.0f};
  if (!masks || masks[e]) {
    const float d0 = dirs[e * 3], d1 = dirs[e * 3 + 1], d2 = dirs[e * 3 + 2];
    const float* co = sc + t * PW;
    float basis[A];
    sh_basis<DEG>(d0, d1, d2, basis);
    const float norm = sqrtf(d0 * d0 + d1 * d1 + d2 * d2);
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
      float result = kC0 * co[ch];
      if (DEG >= 1 && norm != 0.0f) {
        const float x = d0 / norm, y = d1 / norm, z = d2 / norm;
        result += kC1 * (-y * co[3 + ch] + z * co[6 + ch] - x * co[9 + ch]);
#pragma unroll
        for (int l = 2; l <= DEG; ++l) {
          float band = basis[l * l] * co[l * l * 3 + ch];
#pragma unroll
          for (int b = l * l + 1; b < (l + 1) * (l + 1); ++b) band += basis[b] * co[b * 3 + ch];
          result += band;
        }
      }
      out[ch] = result;
    }
  }
  colors[e * 3] = out[0];
  colors[e * 3 + 1] = out[1];
  colors[e * 3 + 2] = out[2];
}

// gsplat_spherical_harmonics.cpp:288-425
template <int DEG, class Co>
__device__ __forceinline__ void sh_dir_vjp(const float dir[3], const Co& co, const float vc[3], float v_dir[3]) {
  v_dir[0] = v_dir[1] = v_dir[2] = 0.0f;
  if (DEG < 1) return;
  const float norm = sqrtf(dir[0] * dir[0] + dir[1] * dir[1] + dir[2] * dir[2]);
  if (norm == 0.0f) return;
  const float inorm = 1.0f / norm;
  const float x = dir[0] * inorm, y = dir[1] * inorm, z = dir[2] * inorm;
  constexpr int A = (DEG + 1) * (DEG + 1);
  float dx[A], dy[A], dz[A];
#pragma unroll
  for (int i = 0; i < A; ++i) dx[i] = dy[i] = dz[i] = 0.0f;
  dx[3] = -kC1;
  dy[1] = -kC1;
  dz[2] = kC1;
  const float z2 = z * z;
  const float f_tmp0_b = -1.092548430592079f * z;
  const float f_c1 = x * x - y * y;
  const float f_s1 = 2.0f * x * y;
  const float f_tmp0_b_z = -1.092548430592079f;
  const float f_c1_x = 2.0f * x, f_c1_y = -2.0f * y;
  const float f_s1_x = 2.0f * y, f_s1_y = 2.0f * x;
  const float p_sh6_z = 2.0f * 0.9461746957575601f * z;
  if constexpr (DEG >= 2) {
    dx[4] = 0.5462742152960395f * f_s1_x;
    dy[4] = 0.5462742152960395f * f_s1_y;
    dy[5] = f_tmp0_b;
    dz[5] = f_tmp0_b_z * y;
    dz[6] = p_sh6_z;
    dx[7] = f_tmp0_b;
    dz[7] = f_tmp0_b_z * x;
    dx[8] = 0.5462742152960395f * f_c1_x;
    dy[8] = 0.5462742152960395f * f_c1_y;
  }
  const float f_tmp0_c = -2.285228997322329f * z2 + 0.4570457994644658f;
  const float f_tmp1_b = 1.445305721320277f * z;
  const float f_c2 = x * f_c1 - y * f_s1;
  const float f_s2 = x * f_s1 + y * f_c1;
  const float p_sh12 = z * (1.865881662950577f * z2 - 1.119528997770346f);
  const float f_tmp0_c_z = -2.285228997322329f * 2.0f * z;
  const float f_tmp1_b_z = 1.445305721320277f;
  const float f_c2_x = f_c1 + x * f_c1_x - y * f_s1_x;
  const float f_c2_y = x * f_c1_y - f_s1 - y * f_s1_y;
  const float f_s2_x = f_s1 + x * f_s1_x + y * f_c1_x;
  const float f_s2_y = x * f_s1_y + f_c1 + y * f_c1_y;
  const float p_sh12_z = 3.0f * 1.865881662950577f * z2 - 1.119528997770346f;
  if constexpr (DEG >= 3) {
    dx[9] = -0.5900435899266435f * f_s2_x;
    dy[9] = -0.5900435899266435f * f_s2_y;
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
    dx[15] = -0.5900435899266435f * f_c2_x;
    dy[15] = -0.5900435899266435f * f_c2_y;
  }
  if constexpr (DEG >= 4) {
    const float f_tmp0_d = z * (-4.683325804901025f * z2 + 2.007139630671868f);
    const float f_tmp1_c = 3.31161143515146f * z2 - 0.47308734787878f;
    const float f_tmp2_b = -1.770130769779931f * z;
    const float f_tmp0_d_z = 3.0f * -4.683325804901025f * z2 + 2.007139630671868f;
    const float f_tmp1_c_z = 2.0f * 3.31161143515146f * z;
    const float f_tmp2_b_z = -1.770130769779931f;
    const float f_c3_x = f_c2 + x * f_c2_x - y * f_s2_x;
    const float f_c3_y = x * f_c2_y - f_s2 - y * f_s2_y;
    const float f_s3_x = f_s2 + y * f_c2_x + x * f_s2_x;
    const float f_s3_y = x * f_s2_y + f_c2 + y * f_c2_y;
    dx[16] = 0.6258357354491763f * f_s3_x;
    dy[16] = 0.6258357354491763f * f_s3_y;
    dx[17] = f_tmp2_b * f_s2_x;
    dy[17] = f_tmp2_b * f_s2_y;
    dz[17] = f_tmp2_b_z * f_s2;
    dx[18] = f_tmp1_c * f_s1_x;
    dy[18] = f_tmp1_c * f_s1_y;
    dz[18] = f_tmp1_c_z * f_s1;
    dy[19] = f_tmp0_d;
    dz[19] = f_tmp0_d_z * y;
    dz[20] = 1.984313483298443f * (p_sh12 + z * p_sh12_z) - 1.006230589874905f * p_sh6_z;
    dx[21] = f_tmp0_d;
    dz[21] = f_tmp0_d_z * x;
    dx[22] = f_tmp1_c * f_c1_x;
    dy[22] = f_tmp1_c * f_c1_y;
    dz[22] = f_tmp1_c_z * f_c1;
    dx[23] = f_tmp2_b * f_c2_x;
    dy[23] = f_tmp2_b * f_c2_y;
    dz[23] = f_tmp2_b_z * f_c2;
    dx[24] = 0.6258357354491763f * f_c3_x;
    dy[24] = 0.6258357354491763f * f_c3_y;
  }
  float vn[3] = {0.0f, 0.0f, 0.0f};
#pragma clang loop unroll(full)
  for (int b = 1; b < A; ++b) {
    const float vb = co[b * 3] * vc[0] + co[b * 3 + 1] * vc[1] + co[b * 3 + 2] * vc[2];
    vn[0] += dx[b] * vb;
    vn[1] += dy[b] * vb;
    vn[2] += dz[b] * vb;
  }
  const float dot = vn[0] * x + vn[1] * y + vn[2] * z;
  v_dir[0] = (vn[0] - dot * x) * inorm;
  v_dir[1] = (vn[1] - dot * y) * inorm;
  v_dir[2] = (vn[2] - dot * z) * inorm;
}

template <int DEG>
__global__ void __launch_bounds__(kShBlock) sh_bwd_kernel(const float* __restrict__ dirs,
                                                          const float* __restrict__ coeffs,
                                                          const uint8_t* __restrict__ masks,
                                                          const float* __restrict__ v_colors, int64_t n, int64_t K,
                                                          uint32_t k3_magic, float* __restrict__ v_dirs,
                                                          float* __restrict__ v_coeffs) {
  constexpr int A = (DEG + 1) * (DEG + 1);
  constexpr int PW = padded(A * 3);
  constexpr int SB = padded(A + 3);
  __shared__ float sc[DEG >= 1 ? kShBlock * PW : 1];
  __shared__ float sb[kShBlock * SB];  // per-lane basis (A) then v_color (3)
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kShBlock;
  const int cnt = static_cast<int>(min<int64_t>(kShBlock, n - e0));
  const int t = threadIdx.x;
  if (v_dirs && DEG >= 1) stage_rows<A>(sc, coeffs + e0 * K * 3, cnt, static_cast<uint32_t>(K * 3), k3_magic);
  float* my = sb + t * SB;
  bool on = false;
  float dir[3] = {0.0f, 0.0f, 0.0f};
  float vc[3] = {0.0f, 0.0f, 0.0f};
  if (t < cnt) {
    const int64_t e = e0 + t;
    on = !masks || masks[e];
    dir[0] = dirs[e * 3];
    dir[1] = dirs[e * 3 + 1];
    dir[2] = dirs[e * 3 + 2];
    vc[0] = v_colors[e * 3];
    vc[1] = v_colors[e * 3 + 1];
    vc[2] = v_colors[e * 3 + 2];
    float basis[A];
    sh_basis<DEG>(dir[0], dir[1], dir[2], basis);
#pragma unroll
    for (int b = 0; b < A; ++b) my[b] = on ? basis[b] : 0.0f;
    my[A] = vc[0];
    my[A + 1] = vc[1];
    my[A + 2] = vc[2];
  }
  __syncthreads();
  if (t < cnt && v_dirs) {
    const int64_t e = e0 + t;
    float vd[3] = {0.0f, 0.0f, 0.0f};
    if (on && DEG >= 1) sh_dir_vjp<DEG>(dir, sc + t * PW, vc, vd);
    v_dirs[e * 3] = vd[0];
    v_dirs[e * 3 + 1] = vd[1];
    v_dirs[e * 3 + 2] = vd[2];
  }
  // Coalesced write of the [cnt, K, 3] slab of v_coeffs (16-byte stores when
  // aligned).
  const uint32_t K3 = static_cast<uint32_t>(K * 3);
  const uint32_t total = static_cast<uint32_t>(cnt) * K3;
  float* out = v_coeffs + e0 * K * 3;
  auto value = [&](uint32_t i) {
    const uint32_t r = fast_div(i, k3_magic);
    const uint32_t c = i - r * K3;
    const uint32_t b = c / 3u;
    const uint32_t ch = c - b * 3u;
    const float* row = sb + r * SB;
    return b < static_cast<uint32_t>(A) ? row[b] * row[A + ch] : 0.0f;
  };
  if ((reinterpret_cast<uintptr_t>(out) & 15) == 0 && (total & 3) == 0) {
    float4* out4 = reinterpret_cast<float4*>(out);
#pragma unroll 2
    for (uint32_t i = t; i < (total >> 2); i += kShBlock)
      out4[i] = make_float4(value(4 * i), value(4 * i + 1), value(4 * i + 2), value(4 * i + 3));
  } else {
    for (uint32_t i = t; i < total; i += kShBlock) out[i] = value(i);
  }
}

// ---------------------------------------------------------------------------
// Camera colours from SH fused with the caller's glue
// (scanner_points_training_utils.py:1005-1034): for every camera c with
// world-to-camera matrix [R | t] and centre campos[c] = -R^T t,
//   d = means - campos[c],  n = d / max(|d|, 1e-8),
//   colors[c] = clamp(SH(n; [dc, rest[:A-1]]) + 0.5, 0, 1),
// without materialising the concatenated and camera-broadcast [C, N, K, 3]
// coefficients. The SH evaluation is the same code and operation order as
// sh_fwd_kernel. The backward recomputes the pre-clamp colour, passes the
// gradient where 0 < colour + 0.5 < 1 (the reference's mx.clip is
// minimum(maximum(x, 0), 1), whose VJPs give a tie to the bound), and sums the
// coefficient and mean gradients over cameras in registers (no atomics).

// Copies `cnt` rows of W floats (global row stride k3 floats, one contiguous
// span) into LDS rows of stride PW at column offset `col0`.
template <int W, int PW>
__device__ __forceinline__ void stage_cols(float* __restrict__ lds, int col0, const float* __restrict__ src, int cnt,
                                           uint32_t k3, uint32_t k3_magic) {
  const uint32_t total = static_cast<uint32_t>(cnt) * k3;
  auto put = [&](uint32_t f, float v) {
    const uint32_t r = fast_div(f, k3_magic);
    const uint32_t c = f - r * k3;
    if (c < static_cast<uint32_t>(W)) lds[r * PW + col0 + c] = v;
  };
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0 && (total & 3) == 0) {
    const float4* src4 = reinterpret_cast<const float4*>(src);
    const uint32_t total4 = total >> 2;
#pragma unroll 4
    for (uint32_t i = threadIdx.x; i < total4; i += kShBlock) {
      const float4 v = src4[i];
      put(4 * i, v.x);
      put(4 * i + 1, v.y);
      put(4 * i + 2, v.z);
      put(4 * i + 3, v.w);
    }
  } else {
#pragma unroll 4
    for (uint32_t i = threadIdx.x; i < total; i += kShBlock) put(i, src[i]);
  }
}

// Colour of coefficient row `co` ([A][3]: an LDS pointer or a register
// array) at direction d; sh_fwd_kernel's per-channel arithmetic. Loops are
// fully unrolled so a register array is never indexed dynamically.
template <int DEG, class Co>
__device__ __forceinline__ void sh_eval(const float d[3], const Co& co, float out[3]) {
  constexpr int A = (DEG + 1) * (DEG + 1);
  float basis[A];
  sh_basis<DEG>(d[0], d[1], d[2], basis);
  const float norm = sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
#pragma clang loop unroll(full)
  for (int ch = 0; ch < 3; ++ch) {
    float result = kC0 * co[ch];
    if (DEG >= 1 && norm != 0.0f) {
      const float x = d[0] / norm, y = d[1] / norm, z = d[2] / norm;
      result += kC1 * (-y * co[3 + ch] + z * co[6 + ch] - x * co[9 + ch]);
#pragma clang loop unroll(full)
      for (int l = 2; l <= DEG; ++l) {
        float band = basis[l * l] * co[l * l * 3 + ch];
#pragma clang loop unroll(full)
        for (int b = l * l + 1; b < (l + 1) * (l + 1); ++b) band += basis[b] * co[b * 3 + ch];
        result += band;
      }
    }
    out[ch] = result;
  }
}

// Camera centre of world-to-camera matrix vm (row-major 4x4, [R | t]):
// -R^T t, as camera_center_from_viewmat (scanner_points_training_utils.py:1005-1008).
__device__ __forceinline__ void camera_centre(const float* __restrict__ vm, float cp[3]) {
#pragma unroll
  for (int i = 0; i < 3; ++i) cp[i] = -((vm[i] * vm[3] + vm[4 + i] * vm[7]) + vm[8 + i] * vm[11]);
}

// The caller's view direction: n = d / max(|d|, 1e-8) (NaN propagates as in
// torch.clamp). Returns |d|.
__device__ __forceinline__ float view_dir(const float* __restrict__ m, const float cp[3], float d[3], float n[3]) {
  d[0] = m[0] - cp[0];
  d[1] = m[1] - cp[1];
  d[2] = m[2] - cp[2];
  const float norm = sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
  const float sc = norm < 1.0e-8f ? 1.0e-8f : norm;
  n[0] = d[0] / sc;
  n[1] = d[1] / sc;
  n[2] = d[2] / sc;
  return norm;
}

// Adds the gradient through n = d / max(|d|, 1e-8) of v_n to v_d (the
// gradient of the means).
__device__ __forceinline__ void view_dir_vjp(const float vn[3], const float n[3], float norm, float vd[3]) {
  if (norm >= 1.0e-8f) {
    const float dot = vn[0] * n[0] + vn[1] * n[1] + vn[2] * n[2];
    vd[0] += (vn[0] - n[0] * dot) / norm;
    vd[1] += (vn[1] - n[1] * dot) / norm;
    vd[2] += (vn[2] - n[2] * dot) / norm;
  } else {
    vd[0] += vn[0] / 1.0e-8f;
    vd[1] += vn[1] / 1.0e-8f;
    vd[2] += vn[2] / 1.0e-8f;
  }
}

__device__ __forceinline__ float clamp01(float x) { return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x); }

// Whether some camera sees Gaussian n of batch b: both radii positive in at
// least one of the C cameras (radii [B, C, N, 2], the projection's output).
// A Gaussian no camera sees has no tile (gsplat_intersect.cpp:74-76 gives it
// none), so the rasterizer never reads its colour and its colour gradient
// is zero.
__device__ __forceinline__ bool seen_by_any(const int32_t* __restrict__ radii, int64_t b, int64_t C, int64_t N,
                                            int64_t n) {
  bool seen = false;
  for (int64_t c = 0; c < C; ++c) {
    const int32_t* r = radii + ((b * C + c) * N + n) * 2;  // 4-byte aligned only
    seen = seen | ((r[0] > 0) & (r[1] > 0));
  }
  return seen;
}

// radii: rows no camera sees get colour 0; PK: colours go to the pairs'
// packed rows (packed_ranks.hpp), pairs without one write nothing.
template <int DEG, bool PK>
__global__ void __launch_bounds__(kShBlock) sh_cam_fwd_kernel(const float* __restrict__ means,
                                                              const float* __restrict__ viewmats,
                                                              const float* __restrict__ dc,
                                                              const float* __restrict__ rest,
                                                              const int32_t* __restrict__ radii, PackedRanks pk,
                                                              int64_t nnz, int64_t C, int64_t N, int64_t R,
                                                              uint32_t r3_magic, float* __restrict__ colors) {
  constexpr int A = (DEG + 1) * (DEG + 1);
  constexpr int PW = padded(A * 3);
  __shared__ float sc[kShBlock * PW];
  const int64_t b = blockIdx.y;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kShBlock;
  const int cnt = static_cast<int>(min<int64_t>(kShBlock, N - e0));
  const int t = threadIdx.x;
  if constexpr (A > 1)
    stage_cols<(A - 1) * 3, PW>(sc, 3, rest + (b * N + e0) * R * 3, cnt, static_cast<uint32_t>(R * 3), r3_magic);
  if (t < cnt) {
    const int64_t g = b * N + e0 + t;
    sc[t * PW] = dc[g * 3];
    sc[t * PW + 1] = dc[g * 3 + 1];
    sc[t * PW + 2] = dc[g * 3 + 2];
  }
  __syncthreads();
  if (t >= cnt) return;
  const int64_t g = b * N + e0 + t;
  const float* co = sc + t * PW;
  const bool live = PK || !radii || seen_by_any(radii, b, C, N, e0 + t);
  for (int64_t c = 0; c < C; ++c) {
    float* out = colors + ((b * C + c) * N + e0 + t) * 3;
    if constexpr (PK) {
      const int64_t rc = packed_row(pk.mask, pk.prefix, (b * C + c) * N + e0 + t, nnz);
      if (rc < 0) continue;
      out = colors + rc * 3;
    }
    if (!live) {
      out[0] = out[1] = out[2] = 0.0f;
      continue;
    }
    float cp[3];
    camera_centre(viewmats + (b * C + c) * 16, cp);
    float d[3], n[3], raw[3];
    view_dir(means + g * 3, cp, d, n);
    sh_eval<DEG>(n, co, raw);
    out[0] = clamp01(raw[0] + 0.5f);
    out[1] = clamp01(raw[1] + 0.5f);
    out[2] = clamp01(raw[2] + 0.5f);
  }
}

// PK: v_colors holds the packed rows, read at each pair's row (pairs
// without one have a zero cotangent).
template <int DEG, bool PK>
__global__ void __launch_bounds__(kShBlock) sh_cam_bwd_kernel(const float* __restrict__ means,
                                                              const float* __restrict__ viewmats,
                                                              const float* __restrict__ dc,
                                                              const float* __restrict__ rest,
                                                              const float* __restrict__ v_colors, PackedRanks pk,
                                                              int64_t nnz, int64_t C, int64_t N,
                                                              int64_t R, uint32_t r3_magic,
                                                              float* __restrict__ v_means, float* __restrict__ v_dc,
                                                              float* __restrict__ v_rest) {
  constexpr int A = (DEG + 1) * (DEG + 1);
  constexpr int PW = padded(A * 3);
  __shared__ float sc[kShBlock * PW];
  const int64_t b = blockIdx.y;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kShBlock;
  const int cnt = static_cast<int>(min<int64_t>(kShBlock, N - e0));
  const int t = threadIdx.x;
  if constexpr (A > 1)
    stage_cols<(A - 1) * 3, PW>(sc, 3, rest + (b * N + e0) * R * 3, cnt, static_cast<uint32_t>(R * 3), r3_magic);
  if (t < cnt) {
    const int64_t g = b * N + e0 + t;
    sc[t * PW] = dc[g * 3];
    sc[t * PW + 1] = dc[g * 3 + 1];
    sc[t * PW + 2] = dc[g * 3 + 2];
  }
  __syncthreads();
  float vco[A * 3];
#pragma unroll
  for (int i = 0; i < A * 3; ++i) vco[i] = 0.0f;
  float vm[3] = {0.0f, 0.0f, 0.0f};
  if (t < cnt) {
    const int64_t g = b * N + e0 + t;
    float* co = sc + t * PW;
    for (int64_t c = 0; c < C; ++c) {
      float cp[3];
    camera_centre(viewmats + (b * C + c) * 16, cp);
      float d[3], n[3], raw[3];
      const float norm = view_dir(means + g * 3, cp, d, n);
      sh_eval<DEG>(n, co, raw);
      const float* vc = v_colors + ((b * C + c) * N + e0 + t) * 3;
      if constexpr (PK) {
        const int64_t rc = packed_row(pk.mask, pk.prefix, (b * C + c) * N + e0 + t, nnz);
        vc = rc >= 0 ? v_colors + rc * 3 : nullptr;
      }
      float gcol[3];
#pragma unroll
      for (int ch = 0; ch < 3; ++ch) {
        const float x = raw[ch] + 0.5f;
        gcol[ch] = 0.0f;
        if (x > 0.0f && x < 1.0f && (!PK || vc)) gcol[ch] = vc[ch];
      }
      float basis[A];
      sh_basis<DEG>(n[0], n[1], n[2], basis);
#pragma unroll
      for (int k = 0; k < A; ++k) {
        vco[k * 3] += basis[k] * gcol[0];
        vco[k * 3 + 1] += basis[k] * gcol[1];
        vco[k * 3 + 2] += basis[k] * gcol[2];
      }
      if constexpr (DEG >= 1) {
        float vn[3];
        sh_dir_vjp<DEG>(n, co, gcol, vn);
        view_dir_vjp(vn, n, norm, vm);
      }
    }
    v_means[g * 3] = vm[0];
    v_means[g * 3 + 1] = vm[1];
    v_means[g * 3 + 2] = vm[2];
    v_dc[g * 3] = vco[0];
    v_dc[g * 3 + 1] = vco[1];
    v_dc[g * 3 + 2] = vco[2];
    // this lane's coefficient row is no longer read: reuse it for the
    // gradient row
#pragma unroll
    for (int i = 3; i < A * 3; ++i) co[i] = vco[i];
  }
  if (R == 0) return;  // uniform
  __syncthreads();
  // coalesced write of the [cnt, R, 3] slab of v_rest; bases past the active
  // degree get zero
  const uint32_t R3 = static_cast<uint32_t>(R * 3);
  const uint32_t total = static_cast<uint32_t>(cnt) * R3;
  float* out = v_rest + (b * N + e0) * R * 3;
  auto value = [&](uint32_t i) {
    const uint32_t r = fast_div(i, r3_magic);
    const uint32_t c = i - r * R3;
    return c < static_cast<uint32_t>((A - 1) * 3) ? sc[r * PW + 3 + c] : 0.0f;
  };
  if ((reinterpret_cast<uintptr_t>(out) & 15) == 0 && (total & 3) == 0) {
    float4* out4 = reinterpret_cast<float4*>(out);
#pragma unroll 2
    for (uint32_t i = t; i < (total >> 2); i += kShBlock)
      out4[i] = make_float4(value(4 * i), value(4 * i + 1), value(4 * i + 2), value(4 * i + 3));
  } else {
    for (uint32_t i = t; i < total; i += kShBlock) out[i] = value(i);
  }
}

// Slab variant of the camera kernels for the common layout where
// features_rest holds exactly the active bases (R == (degree+1)^2 - 1) and
// the row length R*3 is odd (degrees 0, 1 and 3). The block's rows of rest,
// dc and means are each one contiguous span, copied into LDS unchanged with
// 16-byte loads (no index split); the
// odd row stride keeps a lane-per-row LDS read conflict-free. Each lane then
// holds its Gaussian's coefficients in registers for every camera. Same
// arithmetic as sh_cam_fwd_kernel / sh_cam_bwd_kernel, so results are
// identical.
constexpr int kShSlab = 256;
// rows (and threads) of a backward slab block (128 and 64 measured slower:
// 92.6 and 94.9 against 82 us at a million Gaussians, degree 3)
constexpr int kShBwdRows = 256;

template <int W>
__device__ __forceinline__ void stage_slab(float* __restrict__ dst, const float* __restrict__ src, int cnt) {
  if (cnt == kShBwdRows && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    static_assert((kShBwdRows * W) % 4 == 0, "whole float4s per slab");
    constexpr int T4 = kShBwdRows * W / 4;
    constexpr int PER = (T4 + kShBwdRows - 1) / kShBwdRows;
    const float4* s4 = reinterpret_cast<const float4*>(src);
    float4* d4 = reinterpret_cast<float4*>(dst);
    // global and LDS do not alias: the compiler hoists every load above the stores
#pragma clang loop unroll(full)
    for (int i = 0; i < PER; ++i) {
      const int idx = threadIdx.x + i * kShBwdRows;
      if (idx < T4) d4[idx] = s4[idx];
    }
  } else {
    for (int idx = threadIdx.x; idx < cnt * W; idx += kShBwdRows) dst[idx] = src[idx];
  }
}

// Stages the block's slabs and loads lane t's row [dc, rest] into co.
template <int DEG>
__device__ __forceinline__ void slab_rows(const float* __restrict__ means, const float* __restrict__ dc,
                                          const float* __restrict__ rest, int64_t row0, int cnt, float* s_rest,
                                          float* s_dc, float* s_m, float (&co)[(DEG + 1) * (DEG + 1) * 3],
                                          float (&m)[3]) {
  constexpr int R3 = ((DEG + 1) * (DEG + 1) - 1) * 3;
  if constexpr (R3 > 0) stage_slab<R3>(s_rest, rest + row0 * R3, cnt);
  stage_slab<3>(s_dc, dc + row0 * 3, cnt);
  stage_slab<3>(s_m, means + row0 * 3, cnt);
  __syncthreads();
  const int t = threadIdx.x;
  if (t >= cnt) return;
  co[0] = s_dc[t * 3];
  co[1] = s_dc[t * 3 + 1];
  co[2] = s_dc[t * 3 + 2];
#pragma clang loop unroll(full)
  for (int i = 0; i < R3; ++i) co[3 + i] = s_rest[t * R3 + i];
  m[0] = s_m[t * 3];
  m[1] = s_m[t * 3 + 1];
  m[2] = s_m[t * 3 + 2];
}

// The forward: each wave takes a group of 64 Gaussians, reads the group's
// rest rows with 16-byte loads of its contiguous span, and transposes them to
// a row per lane through its own part of the LDS slab; no block barrier is
// taken (the waves are independent). The launch gives every group a wave; a
// wave of a smaller grid walks groups g, g + stride, ... with the next
// group's rows already loading into registers while it computes (a grid of
// the resident blocks only, walking about five groups per wave, measured
// slower: 49.8 against 47.5 us at a million Gaussians, 307 against 272 us at
// three million and eight cameras). Groups that are partial or whose span is
// not 16-byte aligned read their rows per lane instead.
//
// With radii (the projection's [B, C, N, 2]), rows that no camera sees
// (seen_by_any) are neither read nor evaluated: their colours are written as
// 0, and a float4 of the rest span is loaded only when it holds a float of
// a seen row. The rasterizer reads no such row, so the render is unchanged.
// PK (the packed layout): the rank structure (packed_ranks.hpp) selects the
// pairs instead, and each pair's colour is written at its packed row of
// `colors` ([nnz, 3]); pairs without a row write nothing. With one camera
// the selection (radii, or the pair's rank word and prefix) is loaded one
// group ahead of the rows it selects.
template <int DEG, bool PK>
__global__ void __launch_bounds__(kShSlab) sh_cam_fwd_slab_kernel(const float* __restrict__ means,
                                                                  const float* __restrict__ viewmats,
                                                                  const float* __restrict__ dc,
                                                                  const float* __restrict__ rest,
                                                                  const int32_t* __restrict__ radii,
                                                                  PackedRanks pk, int64_t nnz, int64_t C,
                                                                  int64_t N, float* __restrict__ colors) {
  constexpr int A = (DEG + 1) * (DEG + 1);
  constexpr int R3 = (A - 1) * 3;
  constexpr int T4 = R3 > 0 ? kWave * R3 / 4 : 1;  // float4s of a group's rest span
  constexpr int PER = (T4 + kWave - 1) / kWave;
  static_assert((kWave * R3) % 4 == 0, "whole float4s per group");
  __shared__ __align__(16) float s_rest[R3 > 0 ? kShSlab * R3 : 4];
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int64_t n_groups = (N + kWave - 1) / kWave;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * (kShSlab / kWave);
  const bool select = PK || radii != nullptr;
  float* sw = s_rest + wave * kWave * R3;
  auto span = [&](int64_t grp) { return rest + (b * N + grp * kWave) * R3; };
  auto vec_ok = [&](int64_t grp) {
    return R3 > 0 && N - grp * kWave >= kWave && (reinterpret_cast<uintptr_t>(span(grp)) & 15) == 0;
  };
  // one camera: the selection of this lane's row of a group, held a group
  // ahead (radii, or the rank word and prefix of the pair)
  int2 rad = make_int2(0, 0);
  uint64_t pw = 0;
  int32_t pp = 0;
  auto fetch_sel = [&](int64_t grp) {
    const int64_t n = grp * kWave + lane;
    if (C != 1 || n >= N) return;
    if constexpr (PK) {
      pw = pk.mask[(b * N + n) >> 6];
      pp = pk.prefix[(b * N + n) >> 6];
    } else {
      if (radii) rad = make_int2(radii[(b * N + n) * 2], radii[(b * N + n) * 2 + 1]);
    }
  };
  // the group's rows that some camera sees, as a wave mask (every row
  // without a selection); with one camera it reads what fetch_sel loaded
  // and (PK) leaves the lane's packed row in *row
  auto seen_rows = [&](int64_t grp, int64_t* row) -> uint64_t {
    if (!select) return ~0ull;
    const int64_t n = grp * kWave + lane;
    bool seen = false;
    if (n < N) {
      if constexpr (PK) {
        if (C == 1) {
          const int bit = static_cast<int>((b * N + n) & 63);
          const int64_t r = static_cast<int64_t>(pp) + __popcll(pw & ((1ull << bit) - 1ull));
          seen = ((pw >> bit) & 1ull) && r < nnz;
          *row = seen ? r : -1;
        } else {
          for (int64_t c = 0; c < C; ++c) seen = seen | (packed_row(pk.mask, pk.prefix, (b * C + c) * N + n, nnz) >= 0);
        }
      } else {
        seen = C == 1 ? (rad.x > 0) & (rad.y > 0) : seen_by_any(radii, b, C, N, n);
      }
    }
    return __ballot(seen);
  };
  // the group's rest span (clamped: every lane loads PER float4s of it);
  // float4 j holds floats 4j..4j+3, i.e. rows 4j / R3 and (4j + 3) / R3. A
  // float4 of unseen rows only is read from the span's first float4 instead
  // (the loads stay unconditional; the lanes so redirected share one line)
  // and lands in LDS words no seen row reads.
  auto fetch = [&](int64_t grp, int i, uint64_t seen, int ln) {
    constexpr int RD = R3 > 0 ? R3 : 1;
    const int j = min(ln + i * kWave, T4 - 1);
    const int r0 = (4 * j) / RD, r1 = (4 * j + 3) / RD;
    const bool need = ((seen >> r0) | (seen >> r1)) & 1ull;
    return reinterpret_cast<const float4*>(span(grp))[need ? j : 0];
  };
  // dc and mean of this lane's Gaussian of the group (12 bytes each)
  auto fetch_row = [&](int64_t grp, uint64_t seen, float (&p)[6]) {
    const int64_t g = b * N + grp * kWave + lane;
    const bool active = grp * kWave + lane < N && ((seen >> lane) & 1ull);
#pragma clang loop unroll(full)
    for (int k = 0; k < 3; ++k) {
      p[k] = active ? dc[g * 3 + k] : 0.0f;
      p[3 + k] = active ? means[g * 3 + k] : 0.0f;
    }
  };
  float4 r[PER];
  float p[6];
  uint64_t seen_next = 0;
  int64_t row_next = -1;  // PK, one camera: the lane's packed row
  int64_t grp = static_cast<int64_t>(blockIdx.x) * (kShSlab / kWave) + wave;
  if (grp < n_groups) {
    fetch_sel(grp);
    seen_next = seen_rows(grp, &row_next);
    fetch_row(grp, seen_next, p);
    if (vec_ok(grp)) {
#pragma clang loop unroll(full)
      for (int i = 0; i < PER; ++i) r[i] = fetch(grp, i, seen_next, lane);
    }
    if (grp + stride < n_groups) fetch_sel(grp + stride);
  }
  for (; grp < n_groups; grp += stride) {
    const int64_t w0 = grp * kWave;
    const int rows = static_cast<int>(min<int64_t>(kWave, N - w0));
    const uint64_t seen = seen_next;
    const int64_t row = row_next;
    const bool active = lane < rows;
    const bool live = (seen >> lane) & 1ull;
    float co[A * 3], m[3];
#pragma clang loop unroll(full)
    for (int k = 0; k < 3; ++k) {
      co[k] = p[k];
      m[k] = p[3 + k];
    }
    if constexpr (R3 > 0) {
      if (vec_ok(grp)) {  // wave-uniform
        float4* d4 = reinterpret_cast<float4*>(sw);
#pragma clang loop unroll(full)
        for (int i = 0; i < PER; ++i)
          if (lane + i * kWave < T4) d4[lane + i * kWave] = r[i];
        // the wave's LDS writes before its reads of other lanes' rows
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma clang loop unroll(full)
        for (int i = 0; i < R3; ++i) co[3 + i] = sw[lane * R3 + i];
        // the reads before the next group's writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      } else {
        const float* src = span(grp);
#pragma clang loop unroll(full)
        for (int i = 0; i < R3; ++i) co[3 + i] = active && live ? src[lane * R3 + i] : 0.0f;
      }
    }
    if (grp + stride < n_groups) {  // the next group's loads, in flight during the compute
      seen_next = seen_rows(grp + stride, &row_next);
      fetch_row(grp + stride, seen_next, p);
      if (vec_ok(grp + stride)) {
        // the lane index is opaque here, so the loop does not hoist the
        // float4 indices and their rows (registers held across it)
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma clang loop unroll(full)
        for (int i = 0; i < PER; ++i) r[i] = fetch(grp + stride, i, seen_next, ln);
      }
      if (grp + 2 * stride < n_groups) fetch_sel(grp + 2 * stride);
    }
    if (active && (PK ? live : true)) {
      for (int64_t c = 0; c < C; ++c) {
        float* out;
        if constexpr (PK) {
          const int64_t rc = C == 1 ? row : packed_row(pk.mask, pk.prefix, (b * C + c) * N + w0 + lane, nnz);
          if (rc < 0) continue;
          out = colors + rc * 3;
        } else {
          out = colors + ((b * C + c) * N + w0 + lane) * 3;
          if (!live) {
            out[0] = out[1] = out[2] = 0.0f;
            continue;
          }
        }
        float cp[3];
        camera_centre(viewmats + (b * C + c) * 16, cp);
        float d[3], n[3], raw[3];
        view_dir(m, cp, d, n);
        sh_eval<DEG>(n, co, raw);
        out[0] = clamp01(raw[0] + 0.5f);
        out[1] = clamp01(raw[1] + 0.5f);
        out[2] = clamp01(raw[2] + 0.5f);
      }
    }
  }
}

// PK (the packed layout): v_colors holds the packed rows ([nnz, 3]), read
// at each pair's row through the rank structure; pairs without a row have a
// zero cotangent.
template <int DEG, bool PK>
__global__ void __launch_bounds__(kShBwdRows) sh_cam_bwd_slab_kernel(
    const float* __restrict__ means, const float* __restrict__ viewmats, const float* __restrict__ dc,
    const float* __restrict__ rest, const float* __restrict__ v_colors, PackedRanks pk, int64_t nnz, int64_t C,
    int64_t N, float* __restrict__ v_means, float* __restrict__ v_dc, float* __restrict__ v_rest) {
  constexpr int A = (DEG + 1) * (DEG + 1);
  constexpr int R3 = (A - 1) * 3;
  __shared__ __align__(16) float s_rest[R3 > 0 ? kShBwdRows * R3 : 4];
  __shared__ __align__(16) float s_dc[kShBwdRows * 3];
  __shared__ __align__(16) float s_m[kShBwdRows * 3];
  const int64_t b = blockIdx.y;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kShBwdRows;
  const int cnt = static_cast<int>(min<int64_t>(kShBwdRows, N - e0));
  const int t = threadIdx.x;
  float co[A * 3], m[3];
  slab_rows<DEG>(means, dc, rest, b * N + e0, cnt, s_rest, s_dc, s_m, co, m);
  if (t < cnt) {
    const int64_t g = b * N + e0 + t;
    float vco[A * 3];
#pragma clang loop unroll(full)
    for (int i = 0; i < A * 3; ++i) vco[i] = 0.0f;
    float vm[3] = {0.0f, 0.0f, 0.0f};
    for (int64_t c = 0; c < C; ++c) {
      float cp[3];
    camera_centre(viewmats + (b * C + c) * 16, cp);
      float d[3], n[3], raw[3];
      const float norm = view_dir(m, cp, d, n);
      sh_eval<DEG>(n, co, raw);
      const float* vc = v_colors + ((b * C + c) * N + e0 + t) * 3;
      if constexpr (PK) {
        const int64_t rc = packed_row(pk.mask, pk.prefix, (b * C + c) * N + e0 + t, nnz);
        vc = rc >= 0 ? v_colors + rc * 3 : nullptr;
      }
      float gcol[3];
#pragma clang loop unroll(full)
      for (int ch = 0; ch < 3; ++ch) {
        const float x = raw[ch] + 0.5f;
        gcol[ch] = 0.0f;
        if (x > 0.0f && x < 1.0f && (!PK || vc)) gcol[ch] = vc[ch];
      }
      float basis[A];
      sh_basis<DEG>(n[0], n[1], n[2], basis);
#pragma clang loop unroll(full)
      for (int k = 0; k < A; ++k) {
        vco[k * 3] += basis[k] * gcol[0];
        vco[k * 3 + 1] += basis[k] * gcol[1];
        vco[k * 3 + 2] += basis[k] * gcol[2];
      }
      if constexpr (DEG >= 1) {
        float vn[3];
        sh_dir_vjp<DEG>(n, co, gcol, vn);
        view_dir_vjp(vn, n, norm, vm);
      }
    }
    v_means[g * 3] = vm[0];
    v_means[g * 3 + 1] = vm[1];
    v_means[g * 3 + 2] = vm[2];
    v_dc[g * 3] = vco[0];
    v_dc[g * 3 + 1] = vco[1];
    v_dc[g * 3 + 2] = vco[2];
    // this lane's staged row is no longer read: reuse it for the gradient row
#pragma clang loop unroll(full)
    for (int i = 0; i < R3; ++i) s_rest[t * R3 + i] = vco[3 + i];
  }
  if constexpr (R3 > 0) {
    __syncthreads();
    float* out = v_rest + (b * N + e0) * R3;
    if (cnt == kShBwdRows && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
      float4* o4 = reinterpret_cast<float4*>(out);
      const float4* s4 = reinterpret_cast<const float4*>(s_rest);
      for (int idx = t; idx < kShBwdRows * R3 / 4; idx += kShBwdRows) o4[idx] = s4[idx];
    } else {
      for (int idx = t; idx < cnt * R3; idx += kShBwdRows) out[idx] = s_rest[idx];
    }
  }
}

// The slab kernels need rest rows of exactly the active bases with an odd
// float count (degrees 0, 1, 3); other layouts take the general kernels.
constexpr bool slab_degree(int deg) { return deg == 0 || deg == 1 || deg == 3; }

// pk.mask set: the packed layout (PK kernels; colors / v_colors are the
// nnz packed rows).
template <int DEG, bool PK>
int launch_cam_fwd_t(const float* means, const float* viewmats, const float* dc, const float* rest,
                     const int32_t* radii, PackedRanks pk, int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R,
                     float* colors, hipStream_t s) {
  bool slab = false;
  if constexpr (slab_degree(DEG)) {
    if (R == (DEG + 1) * (DEG + 1) - 1) {
      // a wave per group of 64 Gaussians (waves walk further groups past the
      // grid limit)
      const int64_t blocks = ((N + kWave - 1) / kWave + kShSlab / kWave - 1) / (kShSlab / kWave);
      const dim3 grid(static_cast<unsigned>(std::min<int64_t>(blocks, kMaxGridX)), static_cast<unsigned>(B));
      sh_cam_fwd_slab_kernel<DEG, PK><<<grid, kShSlab, 0, s>>>(means, viewmats, dc, rest, radii, pk, nnz, C, N,
                                                               colors);
      slab = true;
    }
  }
  if (!slab) {
    const dim3 grid(grid_for(N, kShBlock), static_cast<unsigned>(B));
    sh_cam_fwd_kernel<DEG, PK><<<grid, kShBlock, 0, s>>>(means, viewmats, dc, rest, radii, pk, nnz, C, N, R,
                                                         magic_for(static_cast<uint32_t>(R > 0 ? R * 3 : 1)), colors);
  }
  return check_launch("sh_camera_colors_forward");
}

template <int DEG>
int launch_cam_fwd(const float* means, const float* viewmats, const float* dc, const float* rest, const int32_t* radii,
                   PackedRanks pk, int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R, float* colors,
                   hipStream_t s) {
  KernelTimer timer("sh_camera_fwd", s);
  if (pk.mask) return launch_cam_fwd_t<DEG, true>(means, viewmats, dc, rest, nullptr, pk, nnz, B, C, N, R, colors, s);
  return launch_cam_fwd_t<DEG, false>(means, viewmats, dc, rest, radii, pk, nnz, B, C, N, R, colors, s);
}

template <int DEG, bool PK>
int launch_cam_bwd_t(const float* means, const float* viewmats, const float* dc, const float* rest,
                     const float* v_colors, PackedRanks pk, int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R,
                     float* v_means, float* v_dc, float* v_rest, hipStream_t s) {
  bool slab = false;
  if constexpr (slab_degree(DEG)) {
    if (R == (DEG + 1) * (DEG + 1) - 1) {
      const dim3 grid(grid_for(N, kShBwdRows), static_cast<unsigned>(B));
      sh_cam_bwd_slab_kernel<DEG, PK><<<grid, kShBwdRows, 0, s>>>(means, viewmats, dc, rest, v_colors, pk, nnz, C, N,
                                                               v_means, v_dc, v_rest);
      slab = true;
    }
  }
  if (!slab) {
    const dim3 grid(grid_for(N, kShBlock), static_cast<unsigned>(B));
    sh_cam_bwd_kernel<DEG, PK><<<grid, kShBlock, 0, s>>>(means, viewmats, dc, rest, v_colors, pk, nnz, C, N, R,
                                                         magic_for(static_cast<uint32_t>(R > 0 ? R * 3 : 1)), v_means,
                                                         v_dc, v_rest);
  }
  return check_launch("sh_camera_colors_backward");
}

template <int DEG>
int launch_cam_bwd(const float* means, const float* viewmats, const float* dc, const float* rest, const float* v_colors,
                   PackedRanks pk, int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R, float* v_means,
                   float* v_dc, float* v_rest, hipStream_t s) {
  KernelTimer timer("sh_camera_bwd", s);
  if (pk.mask)
    return launch_cam_bwd_t<DEG, true>(means, viewmats, dc, rest, v_colors, pk, nnz, B, C, N, R, v_means, v_dc,
                                       v_rest, s);
  return launch_cam_bwd_t<DEG, false>(means, viewmats, dc, rest, v_colors, pk, nnz, B, C, N, R, v_means, v_dc, v_rest,
                                      s);
}

template <int DEG>
int launch_fwd(const float* dirs, const float* coeffs, const uint8_t* masks, int64_t n, int64_t K, float* colors,
               hipStream_t s) {
  {
    KernelTimer timer("sh_fwd", s);
    sh_fwd_kernel<DEG><<<grid_for(n, kShBlock), kShBlock, 0, s>>>(dirs, coeffs, masks, n, K,
                                                                  magic_for(static_cast<uint32_t>(K * 3)), colors);
  }
  return check_launch("spherical_harmonics_forward");
}

template <int DEG>
int launch_bwd(const float* dirs, const float* coeffs, const uint8_t* masks, const float* v_colors, int64_t n,
               int64_t K, float* v_dirs, float* v_coeffs, hipStream_t s) {
  {
    KernelTimer timer("sh_bwd", s);
    sh_bwd_kernel<DEG><<<grid_for(n, kShBlock), kShBlock, 0, s>>>(dirs, coeffs, masks, v_colors, n, K,
                                                                 magic_for(static_cast<uint32_t>(K * 3)), v_dirs,
                                                                 v_coeffs);
  }
  return check_launch("spherical_harmonics_backward");
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" int gsplat_hip_spherical_harmonics_fwd(int32_t degree, const float* dirs, const float* coeffs,
                                                  const uint8_t* masks, int64_t n, int64_t K, float* colors,
                                                  void* stream) {
  if (degree < 0 || degree > 4) return invalid("spherical_harmonics_forward supports degree 0..4.");
  if (K < (degree + 1) * (degree + 1)) return invalid("coeffs has fewer SH bases than degrees_to_use requires.");
  if (n < 0) return invalid("spherical_harmonics_forward: negative size.");
  if (n == 0) return GSPLAT_OK;
  if (!dirs || !coeffs || !colors) return invalid("spherical_harmonics_forward: null pointer.");
  if (K > 1024) return invalid("spherical_harmonics_forward: K exceeds 1024 bases.");
  hipStream_t s = as_stream(stream);
  switch (degree) {
    case 0: return launch_fwd<0>(dirs, coeffs, masks, n, K, colors, s);
    case 1: return launch_fwd<1>(dirs, coeffs, masks, n, K, colors, s);
    case 2: return launch_fwd<2>(dirs, coeffs, masks, n, K, colors, s);
    case 3: return launch_fwd<3>(dirs, coeffs, masks, n, K, colors, s);
    default: return launch_fwd<4>(dirs, coeffs, masks, n, K, colors, s);
  }
}

extern "C" int gsplat_hip_spherical_harmonics_bwd(int32_t degree, const float* dirs, const float* coeffs,
                                                  const uint8_t* masks, const float* v_colors, int64_t n, int64_t K,
                                                  float* v_dirs, float* v_coeffs, void* stream) {
  if (degree < 0 || degree > 4) return invalid("spherical_harmonics_backward supports degree 0..4.");
  if (K < (degree + 1) * (degree + 1)) return invalid("coeffs has fewer SH bases than degrees_to_use requires.");
  if (n < 0) return invalid("spherical_harmonics_backward: negative size.");
  if (n == 0) return GSPLAT_OK;
  if (!dirs || !coeffs || !v_colors || !v_coeffs) return invalid("spherical_harmonics_backward: null pointer.");
  // The slab index i < kShBlock*K*3 keeps the multiply-high split exact
  // while kShBlock * (3K)^2 < 2^32, i.e. K <= 1024.
  if (K > 1024) return invalid("spherical_harmonics_backward: K exceeds 1024 bases.");
  hipStream_t s = as_stream(stream);
  switch (degree) {
    case 0: return launch_bwd<0>(dirs, coeffs, masks, v_colors, n, K, v_dirs, v_coeffs, s);
    case 1: return launch_bwd<1>(dirs, coeffs, masks, v_colors, n, K, v_dirs, v_coeffs, s);
    case 2: return launch_bwd<2>(dirs, coeffs, masks, v_colors, n, K, v_dirs, v_coeffs, s);
    case 3: return launch_bwd<3>(dirs, coeffs, masks, v_colors, n, K, v_dirs, v_coeffs, s);
    default: return launch_bwd<4>(dirs, coeffs, masks, v_colors, n, K, v_dirs, v_coeffs, s);
  }
}

static int check_cam_args(int32_t degree, int64_t B, int64_t C, int64_t N, int64_t R, const char* what) {
  const std::string w(what);
  if (degree < 0 || degree > 4) return invalid(w + " supports degree 0..4.");
  if (B < 0 || C < 0 || N < 0 || R < 0) return invalid(w + ": negative size.");
  if (R < (degree + 1) * (degree + 1) - 1) return invalid(w + ": features_rest has fewer bases than the degree needs.");
  if (R > 1023) return invalid(w + ": features_rest exceeds 1023 bases.");
  if (B > 65535) return invalid(w + ": batch exceeds 65535.");
  return GSPLAT_OK;
}

static int cam_fwd_impl(const char* what, int32_t degree, const float* means, const float* viewmats,
                        const float* features_dc, const float* features_rest, const int32_t* radii, PackedRanks pk,
                        int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R, float* colors, void* stream) {
  int rc = check_cam_args(degree, B, C, N, R, what);
  if (rc) return rc;
  if (B == 0 || C == 0 || N == 0 || (pk.mask && nnz == 0)) return GSPLAT_OK;
  if (!means || !viewmats || !features_dc || (R > 0 && !features_rest) || !colors)
    return invalid(std::string(what) + ": null pointer.");
  hipStream_t s = as_stream(stream);
  switch (degree) {
    case 0: return launch_cam_fwd<0>(means, viewmats, features_dc, features_rest, radii, pk, nnz, B, C, N, R, colors, s);
    case 1: return launch_cam_fwd<1>(means, viewmats, features_dc, features_rest, radii, pk, nnz, B, C, N, R, colors, s);
    case 2: return launch_cam_fwd<2>(means, viewmats, features_dc, features_rest, radii, pk, nnz, B, C, N, R, colors, s);
    case 3: return launch_cam_fwd<3>(means, viewmats, features_dc, features_rest, radii, pk, nnz, B, C, N, R, colors, s);
    default:
      return launch_cam_fwd<4>(means, viewmats, features_dc, features_rest, radii, pk, nnz, B, C, N, R, colors, s);
  }
}

static int cam_bwd_impl(const char* what, int32_t degree, const float* means, const float* viewmats,
                        const float* features_dc, const float* features_rest, const float* v_colors, PackedRanks pk,
                        int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R, float* v_means, float* v_features_dc,
                        float* v_features_rest, void* stream) {
  int rc = check_cam_args(degree, B, C, N, R, what);
  if (rc) return rc;
  if (B == 0 || N == 0) return GSPLAT_OK;
  if (!means || !features_dc || (R > 0 && (!features_rest || !v_features_rest)) || !v_means || !v_features_dc ||
      (C > 0 && (!viewmats || (!v_colors && !(pk.mask && nnz == 0)))))
    return invalid(std::string(what) + ": null pointer.");
  hipStream_t s = as_stream(stream);
  switch (degree) {
    case 0: return launch_cam_bwd<0>(means, viewmats, features_dc, features_rest, v_colors, pk, nnz, B, C, N, R,
                                     v_means, v_features_dc, v_features_rest, s);
    case 1: return launch_cam_bwd<1>(means, viewmats, features_dc, features_rest, v_colors, pk, nnz, B, C, N, R,
                                     v_means, v_features_dc, v_features_rest, s);
    case 2: return launch_cam_bwd<2>(means, viewmats, features_dc, features_rest, v_colors, pk, nnz, B, C, N, R,
                                     v_means, v_features_dc, v_features_rest, s);
    case 3: return launch_cam_bwd<3>(means, viewmats, features_dc, features_rest, v_colors, pk, nnz, B, C, N, R,
                                     v_means, v_features_dc, v_features_rest, s);
    default: return launch_cam_bwd<4>(means, viewmats, features_dc, features_rest, v_colors, pk, nnz, B, C, N, R,
                                      v_means, v_features_dc, v_features_rest, s);
  }
}

// The rank structure at the start of a packed count workspace for B * C * N
// pairs, or an error (mask left null).
static int cam_packed_ranks(const char* what, const void* count_workspace, size_t count_workspace_bytes, int64_t nnz,
                            int64_t B, int64_t C, int64_t N, PackedRanks* pk) {
  *pk = PackedRanks{nullptr, nullptr};
  if (nnz < 0 || B < 0 || C < 0 || N < 0) return invalid(std::string(what) + ": negative size.");
  const int64_t total = B * C * N;
  if (nnz > total) return invalid(std::string(what) + ": more packed rows than pairs.");
  if (total == 0) return GSPLAT_OK;
  if (!count_workspace || count_workspace_bytes < packed_ranks_bytes(total)) {
    set_error(std::string(what) + ": count workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  *pk = packed_ranks_at(count_workspace, total);
  return GSPLAT_OK;
}

extern "C" int gsplat_hip_sh_camera_colors_fwd(int32_t degree, const float* means, const float* viewmats,
                                               const float* features_dc, const float* features_rest,
                                               const int32_t* radii, int64_t B, int64_t C, int64_t N, int64_t R,
                                               float* colors, void* stream) {
  return cam_fwd_impl("sh_camera_colors_forward", degree, means, viewmats, features_dc, features_rest, radii,
                      PackedRanks{nullptr, nullptr}, 0, B, C, N, R, colors, stream);
}

extern "C" int gsplat_hip_sh_camera_colors_bwd(int32_t degree, const float* means, const float* viewmats,
                                               const float* features_dc, const float* features_rest,
                                               const float* v_colors, int64_t B, int64_t C, int64_t N, int64_t R,
                                               float* v_means, float* v_features_dc, float* v_features_rest,
                                               void* stream) {
  return cam_bwd_impl("sh_camera_colors_backward", degree, means, viewmats, features_dc, features_rest, v_colors,
                      PackedRanks{nullptr, nullptr}, 0, B, C, N, R, v_means, v_features_dc, v_features_rest, stream);
}

extern "C" int gsplat_hip_sh_camera_colors_packed_fwd(int32_t degree, const float* means, const float* viewmats,
                                                      const float* features_dc, const float* features_rest,
                                                      const void* count_workspace, size_t count_workspace_bytes,
                                                      int64_t nnz, int64_t B, int64_t C, int64_t N, int64_t R,
                                                      float* rows, void* stream) {
  const char* what = "sh_camera_colors_packed_forward";
  PackedRanks pk;
  const int rc = cam_packed_ranks(what, count_workspace, count_workspace_bytes, nnz, B, C, N, &pk);
  if (rc || !pk.mask) return rc;
  return cam_fwd_impl(what, degree, means, viewmats, features_dc, features_rest, nullptr, pk, nnz, B, C, N, R, rows,
                      stream);
}

extern "C" int gsplat_hip_sh_camera_colors_packed_bwd(int32_t degree, const float* means, const float* viewmats,
                                                      const float* features_dc, const float* features_rest,
                                                      const void* count_workspace, size_t count_workspace_bytes,
                                                      const float* v_rows, int64_t nnz, int64_t B, int64_t C,
                                                      int64_t N, int64_t R, float* v_means, float* v_features_dc,
                                                      float* v_features_rest, void* stream) {
  const char* what = "sh_camera_colors_packed_backward";
  PackedRanks pk;
  const int rc = cam_packed_ranks(what, count_workspace, count_workspace_bytes, nnz, B, C, N, &pk);
  if (rc) return rc;
  // without pairs (no cameras) the kernels read no rows: every gradient is 0
  return cam_bwd_impl(what, degree, means, viewmats, features_dc, features_rest, v_rows, pk, nnz, B, C, N, R, v_means,
                      v_features_dc, v_features_rest, stream);
}
