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
#include "packed_ranks.hpp"
#include "projection_common.hpp"
#include "scan.hpp"

namespace gsplat_hip {
namespace {

// ACT: quats, scales and opacities hold the raw parameters (quaternions,
// log-scales, opacity logits) and opac_out (if non-null) receives the sigmoid
// opacities, written by the first camera of each batch.
// One (camera, Gaussian) pair: the culling of gsplat_projection.metal:214-339
// and the EWA math of gsplat_projection.cpp:446-521, in the same operation
// order. Shared by the dense kernel and both packed passes, so the packed
// outputs equal the dense ones bit for bit.
struct PairOut {
  bool valid;
  int32_t rx, ry;
  float m2x, m2y, depth, c0, c1, c2, comp;
};

template <bool ACT>
__device__ __forceinline__ PairOut project_pair(const float* __restrict__ means, const float* __restrict__ covars,
                                                const float* __restrict__ quats, const float* __restrict__ scales,
                                                const float* __restrict__ opacities, const CamFrame& f, int64_t g,
                                                const gsplat_projection_params& p) {
  PairOut o = {false, 0, 0, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  // Every input of the pair is loaded before the first test: a culled
  // pair's later loads are wasted, but the tests no longer wait for a
  // second and a third round trip to memory.
  const float mw[3] = {means[g * 3], means[g * 3 + 1], means[g * 3 + 2]};
  float qr[4] = {0.0f, 0.0f, 0.0f, 0.0f}, sr[3] = {0.0f, 0.0f, 0.0f}, cv[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  // the activated projection takes quaternions and log-scales only
  const bool use_covars = !ACT && p.use_covars;
  if (use_covars) {
#pragma unroll
    for (int k = 0; k < 6; ++k) cv[k] = covars[g * 6 + k];
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) qr[k] = quats[g * 4 + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) sr[k] = scales[g * 3 + k];
  }
  const float op_in = p.use_opacities ? opacities[g] : 0.0f;
  float mc[3];
  world_to_cam(f, mw, mc);
  bool valid = !(mc[2] < p.near_plane || mc[2] > p.far_plane);
  if (!valid) return o;
  Mat3 cw;
  if (use_covars) {
    cw = read_covar(cv);
  } else {
    float q[4], s[3];
    quat_scale_of<ACT>(qr, sr, q, s);
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
    float op = ACT ? sigmoid_of(op_in) : op_in;
    if (p.calc_compensations) op *= comp;
    valid = !(op < kAlphaThreshold);
    if (valid) extend = fminf(kGaussianExtend, sqrtf(2.0f * logf(op / kAlphaThreshold)));
  }
  if (!valid) return o;
  const float rx = ceilf(extend * sqrtf(cov2d[0]));
  const float ry = ceilf(extend * sqrtf(cov2d[3]));
  valid = !(rx <= p.radius_clip && ry <= p.radius_clip) &&
          !(m2[0] + rx <= 0.0f || m2[0] - rx >= static_cast<float>(p.image_width) || m2[1] + ry <= 0.0f ||
            m2[1] - ry >= static_cast<float>(p.image_height));
  if (!valid) return o;
  const float inv_det = 1.0f / det;
  o.valid = true;
  o.rx = static_cast<int32_t>(rx);
  o.ry = static_cast<int32_t>(ry);
  o.m2x = m2[0];
  o.m2y = m2[1];
  o.depth = mc[2];
  o.c0 = cov2d[3] * inv_det;
  o.c1 = -cov2d[1] * inv_det;
  o.c2 = cov2d[0] * inv_det;
  o.comp = comp;
  return o;
}

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
  // the logit is loaded with the pair's inputs, its sigmoid stored after
  const bool write_opac = ACT && opac_out && cam == b * C;
  const float logit = write_opac ? opacities[g] : 0.0f;
  const PairOut o = project_pair<ACT>(means, covars, quats, scales, opacities, f, g, p);
  if (write_opac) opac_out[g] = sigmoid_of(logit);
  radii[idx * 2] = o.rx;
  radii[idx * 2 + 1] = o.ry;
  means2d[idx * 2] = o.m2x;
  means2d[idx * 2 + 1] = o.m2y;
  depths[idx] = o.depth;
  conics[idx * 3] = o.c0;
  conics[idx * 3 + 1] = o.c1;
  conics[idx * 3 + 2] = o.c2;
  if (compensations) compensations[idx] = o.comp;
}

// ---------------------------------------------------------------------------
// Packed layout (upstream gsplat's fully_fused_projection(packed=True),
// note/gsplat_cuda_source_map.md:273-315): only the visible pairs, in flat
// order idx = (b * C + c) * N + n. Pass 1 computes every pair's visibility
// and stores one bit per pair (a 64-bit word per wave of 64 consecutive idx)
// with the word's popcount; an exclusive scan of the popcounts gives each
// word's first packed position; pass 2 recomputes the visible pairs and
// writes them at prefix[word] + popcount(bits below). The same bit words and
// prefixes ("rank structure", 3/16 byte per pair) let the backward find a
// pair's packed row without a dense index map.

// ACT: raw parameters, as the activated projection (project_pair<true>).
template <bool ACT>
__global__ void __launch_bounds__(kProjBlock) projection_packed_mask_kernel(
    const float* __restrict__ means, const float* __restrict__ covars, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ opacities, const float* __restrict__ viewmats,
    const float* __restrict__ Ks, int64_t C, int64_t N, int64_t total, gsplat_projection_params p,
    uint64_t* __restrict__ mask, int32_t* __restrict__ word_counts) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kProjBlock + threadIdx.x;
  bool valid = false;
  if (idx < total) {
    const int64_t cam = idx / N, n = idx - cam * N;
    const CamFrame f = load_camera(viewmats + cam * 16, Ks + cam * 9);
    valid = project_pair<ACT>(means, covars, quats, scales, opacities, f, (cam / C) * N + n, p).valid;
  }
  const uint64_t bits = __ballot(valid);
  if ((threadIdx.x % kWave) == 0 && idx < total) {
    mask[idx >> 6] = bits;
    word_counts[idx >> 6] = __popcll(bits);
  }
}

// ACT: raw parameters; opac_rows (if non-null) receives each visible pair's
// sigmoid opacity (the rasterizer's per-row opacities).
template <bool ACT>
__global__ void __launch_bounds__(kProjBlock) projection_packed_write_kernel(
    const float* __restrict__ means, const float* __restrict__ covars, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ opacities, const float* __restrict__ viewmats,
    const float* __restrict__ Ks, int64_t C, int64_t N, int64_t total, gsplat_projection_params p,
    const uint64_t* __restrict__ mask, const int32_t* __restrict__ prefix, int64_t nnz,
    int32_t* __restrict__ batch_ids, int32_t* __restrict__ camera_ids, int32_t* __restrict__ gaussian_ids,
    int32_t* __restrict__ radii, float* __restrict__ means2d, float* __restrict__ depths,
    float* __restrict__ conics, float* __restrict__ compensations, float* __restrict__ opac_rows) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kProjBlock + threadIdx.x;
  if (idx >= total || !((mask[idx >> 6] >> (idx & 63)) & 1ull)) return;
  const int64_t pos = packed_rank(mask, prefix, idx);
  if (pos >= nnz) return;  // nnz smaller than the count: keep writes in bounds
  const int64_t cam = idx / N, n = idx - cam * N;
  const int64_t b = cam / C;
  const CamFrame f = load_camera(viewmats + cam * 16, Ks + cam * 9);
  const PairOut o = project_pair<ACT>(means, covars, quats, scales, opacities, f, b * N + n, p);
  if constexpr (ACT) {
    if (opac_rows) opac_rows[pos] = sigmoid_of(opacities[b * N + n]);
  }
  batch_ids[pos] = static_cast<int32_t>(b);
  camera_ids[pos] = static_cast<int32_t>(cam - b * C);
  gaussian_ids[pos] = static_cast<int32_t>(n);
  radii[pos * 2] = o.rx;
  radii[pos * 2 + 1] = o.ry;
  means2d[pos * 2] = o.m2x;
  means2d[pos * 2 + 1] = o.m2y;
  depths[pos] = o.depth;
  conics[pos * 3] = o.c0;
  conics[pos * 3 + 1] = o.c1;
  conics[pos * 3 + 2] = o.c2;
  if (compensations) compensations[pos] = o.comp;
}

// indptr[cam] = packed position of the first pair of camera cam (B*C + 1
// entries; the last is nnz, read from nnz_dev when that is non-null).
__global__ void __launch_bounds__(256) projection_packed_indptr_kernel(const uint64_t* __restrict__ mask,
                                                                       const int32_t* __restrict__ prefix,
                                                                       int64_t n_cams, int64_t N, int64_t nnz,
                                                                       const int64_t* __restrict__ nnz_dev,
                                                                       int32_t* __restrict__ indptr) {
  const int64_t cam = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (cam > n_cams) return;
  const int64_t nn = nnz_dev ? *nnz_dev : nnz;
  indptr[cam] = static_cast<int32_t>(cam == n_cams ? nn : min<int64_t>(packed_rank(mask, prefix, cam * N), nn));
}

// Backward: bit per pair from the packed (batch, camera, gaussian) ids.
__global__ void __launch_bounds__(256) projection_packed_scatter_kernel(const int32_t* __restrict__ batch_ids,
                                                                        const int32_t* __restrict__ camera_ids,
                                                                        const int32_t* __restrict__ gaussian_ids,
                                                                        int64_t nnz, int64_t B, int64_t C, int64_t N,
                                                                        uint64_t* __restrict__ mask) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int lane = threadIdx.x % kWave;
  int64_t word = -1;
  uint64_t bit = 0;
  if (e < nnz) {
    const int64_t b = batch_ids ? batch_ids[e] : 0, c = camera_ids[e], n = gaussian_ids[e];
    if (b >= 0 && b < B && c >= 0 && c < C && n >= 0 && n < N) {  // others are ignored
      const int64_t idx = (b * C + c) * N + n;
      word = idx >> 6;
      bit = 1ull << (idx & 63);
    }
  }
  // Entries in the forward's order put consecutive lanes on the same word:
  // OR the bits of equal-word lanes together (each lane gathers from the
  // lanes above it with the same word) so that one lane per word and wave
  // issues the atomic instead of up to 64.
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint64_t ob = __shfl_down(bit, off, kWave);
    const int64_t ow = __shfl_down(word, off, kWave);
    if (lane + off < kWave && ow == word) bit |= ob;
  }
  const int64_t prev = __shfl_up(word, 1, kWave);
  if (word >= 0 && (lane == 0 || prev != word))
    atomicOr(reinterpret_cast<unsigned long long*>(mask) + word, bit);
}

__global__ void __launch_bounds__(256) popcount_words_kernel(const uint64_t* __restrict__ mask, int64_t n_words,
                                                             int32_t* __restrict__ counts) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (w < n_words) counts[w] = __popcll(mask[w]);
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
  if (p.camera_model < 0 || p.camera_model > 2) return invalid(op + ": unknown camera model.");
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

// Packed layout workspace: [bit words | word prefixes | scan | view-matrix
// partials (backward with v_viewmats)].
static size_t align256(size_t b) { return (b + 255) / 256 * 256; }

struct PackedLayout {
  uint64_t* mask;
  int32_t* prefix;
  void* scan_ws;
  float* partials;
  int64_t n_words;
};

// The rank structure (packed_ranks.hpp: words, then prefixes) first, then
// the scan's workspace and the view-matrix partials.
static size_t packed_layout(int64_t B, int64_t C, int64_t N, bool vm, PackedLayout* l, void* base) {
  const int64_t total = B * C * N;
  const int64_t nw = (total + 63) / 64;
  const size_t mask_b = packed_ranks_align(static_cast<size_t>(nw) * 8);
  const size_t pre_b = packed_ranks_align(static_cast<size_t>(nw) * 4);
  const size_t scan_b = align256(scan_workspace_bytes(nw));
  const size_t part_b = vm && C > 0 ? static_cast<size_t>(B * C) * grid_for(N, kProjBlock) * 12 * sizeof(float) : 0;
  if (l && base) {
    char* p = static_cast<char*>(base);
    l->mask = reinterpret_cast<uint64_t*>(p);
    l->prefix = reinterpret_cast<int32_t*>(p + mask_b);
    l->scan_ws = p + mask_b + pre_b;
    l->partials = part_b ? reinterpret_cast<float*>(p + mask_b + pre_b + scan_b) : nullptr;
    l->n_words = nw;
  }
  return mask_b + pre_b + scan_b + part_b;
}

static int packed_args(const std::string& op, const float* means, const float* covars, const float* quats,
                       const float* scales, const float* viewmats, const float* Ks, int64_t B, int64_t C, int64_t N,
                       const gsplat_projection_params* params) {
  if (!params) return invalid(op + ": null params.");
  if (B < 0 || C < 0 || N < 0) return invalid(op + ": negative size.");
  // packed rows and word prefixes are int32
  if (B * C * N > static_cast<int64_t>(INT32_MAX)) return invalid(op + ": more than 2^31-1 (camera, Gaussian) pairs.");
  if (B * C * N == 0) return GSPLAT_OK;
  if (!means || !viewmats || !Ks) return invalid(op + ": null pointer.");
  if (params->use_covars ? !covars : (!quats || !scales)) return invalid(op + " expects covars or quats+scales.");
  return GSPLAT_OK;
}

extern "C" size_t gsplat_hip_projection_packed_workspace_size(int64_t B, int64_t C, int64_t N, int32_t viewmats_grad) {
  if (B <= 0 || C <= 0 || N <= 0) return 0;
  return packed_layout(B, C, N, viewmats_grad != 0, nullptr, nullptr);
}

// The packed passes of the operator (ACT false) and of the activated
// projection (ACT true: quats, scales, opacities hold raw quaternions,
// log-scales and opacity logits; the forward also writes the per-row sigmoid
// opacities, the backward reads the count pass's rank structure from
// rank_ws instead of rebuilding it from the ids, and its opacity cotangent
// is per row).
template <bool ACT>
int packed_count_impl(const std::string& op, const float* means, const float* covars, const float* quats,
                      const float* scales, const float* opacities, const float* viewmats, const float* Ks, int64_t B,
                      int64_t C, int64_t N, const gsplat_projection_params* params, int64_t* nnz_dev,
                      void* workspace, size_t workspace_bytes, void* stream) {
  int rc = packed_args(op, means, covars, quats, scales, viewmats, Ks, B, C, N, params);
  if (rc) return rc;
  if (ACT && params->use_covars) return invalid(op + " takes quats and log_scales, not covars.");
  if (!nnz_dev) return invalid(op + ": null count.");
  hipStream_t s = as_stream(stream);
  if (B * C * N == 0) return fill_zero(nnz_dev, sizeof(int64_t), s);
  if (params->use_opacities && !opacities) return invalid(op + ": null opacities.");
  PackedLayout l;
  if (!workspace || workspace_bytes < packed_layout(B, C, N, false, &l, workspace)) {
    set_error(op + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  const int64_t total = B * C * N;
  {
    KernelTimer timer("projection_packed_count", s);
    projection_packed_mask_kernel<ACT><<<grid_for(total, kProjBlock), kProjBlock, 0, s>>>(
        means, covars, quats, scales, opacities, viewmats, Ks, C, N, total, *params, l.mask, l.prefix);
  }
  if ((rc = check_launch(op.c_str()))) return rc;
  return scan_exclusive_i32(l.prefix, l.prefix, l.n_words, nnz_dev, l.scan_ws, s);
}

template <bool ACT>
int packed_fwd_impl(const std::string& op, const float* means, const float* covars, const float* quats,
                    const float* scales, const float* opacities, const float* viewmats, const float* Ks, int64_t B,
                    int64_t C, int64_t N, const gsplat_projection_params* params, int64_t nnz,
                    const int64_t* nnz_dev, int32_t* batch_ids, int32_t* camera_ids, int32_t* gaussian_ids,
                    int32_t* indptr, int32_t* radii, float* means2d, float* depths, float* conics,
                    float* compensations, float* opac_rows, const void* workspace, size_t workspace_bytes,
                    void* stream) {
  int rc = packed_args(op, means, covars, quats, scales, viewmats, Ks, B, C, N, params);
  if (rc) return rc;
  if (ACT && params->use_covars) return invalid(op + " takes quats and log_scales, not covars.");
  if (nnz < 0) return invalid(op + ": negative nnz.");
  hipStream_t s = as_stream(stream);
  const int64_t total = B * C * N;
  if (!indptr) return invalid(op + ": null indptr.");
  if (total == 0) return fill_zero(indptr, (B * C + 1) * sizeof(int32_t), s);
  if (nnz > 0 && (!batch_ids || !camera_ids || !gaussian_ids || !radii || !means2d || !depths || !conics))
    return invalid(op + ": null pointer.");
  if (nnz > 0 && params->calc_compensations && !compensations) return invalid(op + ": null compensations.");
  if (params->use_opacities && !opacities) return invalid(op + ": null opacities.");
  if (ACT && nnz > 0 && opac_rows && !opacities) return invalid(op + ": opacities out without opacity logits.");
  PackedLayout l;
  if (!workspace || workspace_bytes < packed_layout(B, C, N, false, &l, const_cast<void*>(workspace))) {
    set_error(op + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  {
    KernelTimer timer("projection_packed_fwd", s);
    if (nnz > 0)
      projection_packed_write_kernel<ACT><<<grid_for(total, kProjBlock), kProjBlock, 0, s>>>(
          means, covars, quats, scales, opacities, viewmats, Ks, C, N, total, *params, l.mask, l.prefix, nnz,
          batch_ids, camera_ids, gaussian_ids, radii, means2d, depths, conics,
          params->calc_compensations ? compensations : nullptr, ACT ? opac_rows : nullptr);
    projection_packed_indptr_kernel<<<grid_for(B * C + 1, 256), 256, 0, s>>>(l.mask, l.prefix, B * C, N, nnz,
                                                                             nnz_dev, indptr);
  }
  return check_launch(op.c_str());
}

template <bool ACT>
int packed_bwd_impl(const std::string& op, const float* means, const float* covars, const float* quats,
                    const float* scales, const float* viewmats, const float* Ks, int64_t B, int64_t C, int64_t N,
                    const gsplat_projection_params* params, int64_t nnz, const int32_t* batch_ids,
                    const int32_t* camera_ids, const int32_t* gaussian_ids, const void* rank_ws,
                    size_t rank_ws_bytes, const float* conics, const float* compensations, const float* v_means2d,
                    const float* v_depths, const float* v_conics, const float* v_compensations,
                    const float* logits, const float* v_opac_rows, float* v_means, float* v_covars, float* v_quats,
                    float* v_scales, float* v_logits, float* v_viewmats, float* v_viewspace, void* workspace,
                    size_t workspace_bytes, void* stream) {
  int rc = packed_args(op, means, covars, quats, scales, viewmats, Ks, B, C, N, params);
  if (rc) return rc;
  const gsplat_projection_params& p = *params;
  if (ACT && p.use_covars) return invalid(op + " takes quats and log_scales, not covars.");
  if (p.camera_model < 0 || p.camera_model > 2) return invalid(op + ": unknown camera model.");
  if (nnz < 0) return invalid(op + ": negative nnz.");
  hipStream_t s = as_stream(stream);
  if (B * N == 0) {
    if (v_viewmats && B * C > 0) return fill_zero(v_viewmats, B * C * 16 * sizeof(float), s);
    return GSPLAT_OK;
  }
  if (!v_means || (p.use_covars ? !v_covars : (!v_quats || !v_scales))) return invalid(op + ": null pointer.");
  if (nnz > 0 && (!conics || !v_means2d || !v_conics)) return invalid(op + ": null pointer.");
  if (!ACT && v_viewspace) return invalid(op + ": no viewspace gradient here.");
  if (!ACT && nnz > 0 && (!camera_ids || !gaussian_ids)) return invalid(op + ": null pointer.");
  if (!ACT && nnz > 0 && B > 1 && !batch_ids) return invalid(op + ": null batch_ids with more than one batch.");
  if (v_compensations && !compensations) return invalid(op + ": v_compensations without compensations.");
  if (ACT && v_logits && !logits) return invalid(op + ": v_opacity_logits without opacity logits.");
  if (B > 65535) return invalid(op + ": batch exceeds 65535.");
  PackedLayout l;
  if (!workspace || workspace_bytes < packed_layout(B, C, N, v_viewmats != nullptr, &l, workspace)) {
    set_error(op + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  const uint64_t* mask = l.mask;
  const int32_t* prefix = l.prefix;
  if constexpr (ACT) {  // the count pass's rank structure
    PackedLayout r;
    if (!rank_ws || rank_ws_bytes < packed_layout(B, C, N, false, &r, const_cast<void*>(rank_ws))) {
      set_error(op + ": count workspace too small.");
      return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
    }
    mask = r.mask;
    prefix = r.prefix;
  }
  const dim3 grid(grid_for(N, kProjBlock), static_cast<unsigned>(B));
  if constexpr (!ACT) {
    {
      KernelTimer timer("projection_packed_bwd", s);
      if ((rc = fill_zero(l.mask, static_cast<size_t>(l.n_words) * 8, s))) return rc;
      if (nnz > 0)
        projection_packed_scatter_kernel<<<grid_for(nnz, 256), 256, 0, s>>>(batch_ids, camera_ids, gaussian_ids,
                                                                             nnz, B, C, N, l.mask);
      popcount_words_kernel<<<grid_for(l.n_words, 256), 256, 0, s>>>(l.mask, l.n_words, l.prefix);
    }
    if ((rc = check_launch(op.c_str()))) return rc;
    if ((rc = scan_exclusive_i32(l.prefix, l.prefix, l.n_words, nullptr, l.scan_ws, s))) return rc;
  }
  {
    KernelTimer timer("projection_packed_bwd", s);
    launch_projection_bwd(ACT, grid, s, means, covars, quats, scales, viewmats, Ks, C, N, p, nullptr, conics,
                          compensations, v_means2d, v_depths, v_conics, v_compensations, v_means, v_covars, v_quats,
                          v_scales, v_viewmats ? l.partials : nullptr, ACT ? logits : nullptr, nullptr,
                          ACT ? v_logits : nullptr, mask, prefix, ACT ? v_opac_rows : nullptr,
                          ACT ? v_viewspace : nullptr);
  }
  if ((rc = check_launch(op.c_str())) || !v_viewmats) return rc;
  {
    KernelTimer timer("projection_bwd_viewmats", s);
    viewmat_reduce_kernel<<<static_cast<unsigned>(B * C), 256, 0, s>>>(l.partials, static_cast<int>(grid.x),
                                                                       v_viewmats);
  }
  return check_launch(op.c_str());
}

extern "C" int gsplat_hip_projection_packed_count(const float* means, const float* covars, const float* quats,
                                                  const float* scales, const float* opacities, const float* viewmats,
                                                  const float* Ks, int64_t B, int64_t C, int64_t N,
                                                  const gsplat_projection_params* params, int64_t* nnz_dev,
                                                  void* workspace, size_t workspace_bytes, void* stream) {
  return packed_count_impl<false>("projection_ewa_3dgs_packed_forward", means, covars, quats, scales, opacities,
                                  viewmats, Ks, B, C, N, params, nnz_dev, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_projection_packed_fwd(const float* means, const float* covars, const float* quats,
                                                const float* scales, const float* opacities, const float* viewmats,
                                                const float* Ks, int64_t B, int64_t C, int64_t N,
                                                const gsplat_projection_params* params, int64_t nnz,
                                                int32_t* batch_ids, int32_t* camera_ids, int32_t* gaussian_ids,
                                                int32_t* indptr, int32_t* radii, float* means2d, float* depths,
                                                float* conics, float* compensations, const void* workspace,
                                                size_t workspace_bytes, void* stream) {
  return packed_fwd_impl<false>("projection_ewa_3dgs_packed_forward", means, covars, quats, scales, opacities,
                                viewmats, Ks, B, C, N, params, nnz, nullptr, batch_ids, camera_ids, gaussian_ids,
                                indptr, radii, means2d, depths, conics, compensations, nullptr, workspace,
                                workspace_bytes, stream);
}

extern "C" int gsplat_hip_projection_packed_bwd(const float* means, const float* covars, const float* quats,
                                                const float* scales, const float* viewmats, const float* Ks,
                                                int64_t B, int64_t C, int64_t N,
                                                const gsplat_projection_params* params, int64_t nnz,
                                                const int32_t* batch_ids, const int32_t* camera_ids,
                                                const int32_t* gaussian_ids, const float* conics,
                                                const float* compensations, const float* v_means2d,
                                                const float* v_depths, const float* v_conics,
                                                const float* v_compensations, float* v_means, float* v_covars,
                                                float* v_quats, float* v_scales, float* v_viewmats, void* workspace,
                                                size_t workspace_bytes, void* stream) {
  return packed_bwd_impl<false>("projection_ewa_3dgs_packed_backward", means, covars, quats, scales, viewmats, Ks, B,
                                C, N, params, nnz, batch_ids, camera_ids, gaussian_ids, nullptr, 0, conics,
                                compensations, v_means2d, v_depths, v_conics, v_compensations, nullptr, nullptr,
                                v_means, v_covars, v_quats, v_scales, nullptr, v_viewmats, nullptr, workspace,
                                workspace_bytes, stream);
}

extern "C" int gsplat_hip_activated_projection_packed_count(const float* means, const float* quats,
                                                            const float* log_scales, const float* opacity_logits,
                                                            const float* viewmats, const float* Ks, int64_t B,
                                                            int64_t C, int64_t N,
                                                            const gsplat_projection_params* params, int64_t* nnz_dev,
                                                            void* workspace, size_t workspace_bytes, void* stream) {
  return packed_count_impl<true>("activated_projection_packed_forward", means, nullptr, quats, log_scales,
                                 opacity_logits, viewmats, Ks, B, C, N, params, nnz_dev, workspace, workspace_bytes,
                                 stream);
}

extern "C" int gsplat_hip_activated_projection_packed_fwd(
    const float* means, const float* quats, const float* log_scales, const float* opacity_logits,
    const float* viewmats, const float* Ks, int64_t B, int64_t C, int64_t N, const gsplat_projection_params* params,
    int64_t nnz, const int64_t* nnz_dev, int32_t* batch_ids, int32_t* camera_ids, int32_t* gaussian_ids,
    int32_t* indptr, int32_t* radii, float* means2d, float* depths, float* conics, float* compensations,
    float* opacities, const void* workspace, size_t workspace_bytes, void* stream) {
  return packed_fwd_impl<true>("activated_projection_packed_forward", means, nullptr, quats, log_scales,
                               opacity_logits, viewmats, Ks, B, C, N, params, nnz, nnz_dev, batch_ids, camera_ids,
                               gaussian_ids, indptr, radii, means2d, depths, conics, compensations, opacities,
                               workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_activated_projection_packed_bwd(
    const float* means, const float* quats, const float* log_scales, const float* opacity_logits,
    const float* viewmats, const float* Ks, int64_t B, int64_t C, int64_t N, const gsplat_projection_params* params,
    int64_t nnz, const void* count_workspace, size_t count_workspace_bytes, const float* conics,
    const float* compensations, const float* v_means2d, const float* v_depths, const float* v_conics,
    const float* v_compensations, const float* v_opacities, float* v_means, float* v_quats, float* v_log_scales,
    float* v_opacity_logits, float* v_viewmats, float* v_viewspace, void* workspace, size_t workspace_bytes,
    void* stream) {
  return packed_bwd_impl<true>("activated_projection_packed_backward", means, nullptr, quats, log_scales, viewmats,
                               Ks, B, C, N, params, nnz, nullptr, nullptr, nullptr, count_workspace,
                               count_workspace_bytes, conics, compensations, v_means2d, v_depths, v_conics,
                               v_compensations, opacity_logits, v_opacities, v_means, nullptr, v_quats, v_log_scales,
                               v_opacity_logits, v_viewmats, v_viewspace, workspace, workspace_bytes, stream);
}

// Rows of the packed layout <-> dense (batch, camera, Gaussian) slots of K
// floats each: the gather reads each row's slot; the scatter writes every
// slot, the row's values where the pair has one (rank structure of the
// count pass) and zeros elsewhere.
__global__ void __launch_bounds__(256) packed_rows_gather_kernel(const float* __restrict__ dense,
                                                                 const int32_t* __restrict__ batch_ids,
                                                                 const int32_t* __restrict__ camera_ids,
                                                                 const int32_t* __restrict__ gaussian_ids,
                                                                 int64_t nnz, int64_t B, int64_t C, int64_t N,
                                                                 int K, float* __restrict__ rows) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= nnz) return;
  const int64_t b = batch_ids ? batch_ids[r] : 0, c = camera_ids[r], g = gaussian_ids[r];
  const bool ok = b >= 0 && b < B && c >= 0 && c < C && g >= 0 && g < N;
  const float* src = dense + ((ok ? (b * C + c) * N + g : 0)) * K;
  for (int k = 0; k < K; ++k) rows[r * K + k] = ok ? src[k] : 0.0f;
}

__global__ void __launch_bounds__(256) packed_rows_scatter_kernel(const float* __restrict__ rows,
                                                                  const uint64_t* __restrict__ mask,
                                                                  const int32_t* __restrict__ prefix, int64_t nnz,
                                                                  int64_t total, int K, float* __restrict__ dense) {
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (pair >= total) return;
  int64_t r = -1;
  if ((mask[pair >> 6] >> (pair & 63)) & 1ull) {
    r = packed_rank(mask, prefix, pair);
    if (r >= nnz) r = -1;
  }
  for (int k = 0; k < K; ++k) dense[pair * K + k] = r >= 0 ? rows[r * K + k] : 0.0f;
}

extern "C" int gsplat_hip_packed_rows_gather(const float* dense, const int32_t* batch_ids, const int32_t* camera_ids,
                                             const int32_t* gaussian_ids, int64_t nnz, int64_t B, int64_t C,
                                             int64_t N, int32_t K, float* rows, void* stream) {
  if (nnz < 0 || B < 0 || C < 0 || N < 0 || K <= 0) return invalid("packed_rows_gather: invalid sizes.");
  if (nnz == 0) return GSPLAT_OK;
  if (!dense || !camera_ids || !gaussian_ids || !rows) return invalid("packed_rows_gather: null pointer.");
  if (B > 1 && !batch_ids) return invalid("packed_rows_gather: null batch_ids with more than one batch.");
  hipStream_t s = as_stream(stream);
  {
    KernelTimer timer("packed_rows", s);
    packed_rows_gather_kernel<<<grid_for(nnz, 256), 256, 0, s>>>(dense, batch_ids, camera_ids, gaussian_ids, nnz, B,
                                                                  C, N, K, rows);
  }
  return check_launch("packed_rows_gather");
}

extern "C" int gsplat_hip_packed_rows_scatter(const float* rows, const void* count_workspace,
                                              size_t count_workspace_bytes, int64_t nnz, int64_t B, int64_t C,
                                              int64_t N, int32_t K, float* dense, void* stream) {
  if (nnz < 0 || B < 0 || C < 0 || N < 0 || K <= 0) return invalid("packed_rows_scatter: invalid sizes.");
  const int64_t total = B * C * N;
  if (total == 0) return GSPLAT_OK;
  if (!dense || (nnz > 0 && !rows)) return invalid("packed_rows_scatter: null pointer.");
  PackedLayout l;
  if (!count_workspace || count_workspace_bytes < packed_layout(B, C, N, false, &l, const_cast<void*>(count_workspace))) {
    set_error("packed_rows_scatter: count workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  hipStream_t s = as_stream(stream);
  {
    KernelTimer timer("packed_rows", s);
    packed_rows_scatter_kernel<<<grid_for(total, 256), 256, 0, s>>>(rows, l.mask, l.prefix, nnz, total, K, dense);
  }
  return check_launch("packed_rows_scatter");
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
