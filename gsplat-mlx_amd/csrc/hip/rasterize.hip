// Tile rasterization (front-to-back alpha compositing) forward / backward for
// gfx950.
//
// One block per (image, tile) with tile_size^2 lanes, one pixel per lane
// (16x16 tiles -> 4 wave64s, each covering 16x4 pixels). The tile's sorted
// Gaussian list is walked in batches of blockDim entries: each lane gathers
// one Gaussian record (mean, conic, opacity, colors) into LDS, then every
// lane evaluates the whole batch from LDS. Forward stops when every lane of
// the block has saturated (block vote). Backward walks the same lists
// back-to-front from the block's largest last_id, rebuilding transmittance
// per pixel, and reduces each Gaussian's partial gradients across the wave
// with DPP before one atomic per (wave, Gaussian, component); waves where no
// lane contributes skip the reduction.
//
// Per-pixel math follows gsplat_core/gsplat_rasterize.cpp:291-368 (forward)
// and :432-554 (backward) operation for operation; the Gaussian falloff and
// alpha tests are evaluated exactly as the reference (no FMA contraction in
// this file) so compositing decisions match it.
#include "common.hpp"

namespace gsplat_hip {
namespace {

constexpr int kMaxChannels = 64;

struct RasterArgs {
  const float* means2d;
  const float* conics;
  const float* colors;
  const float* opacities;
  const float* backgrounds;
  const uint8_t* masks;
  const int32_t* tile_offsets;
  const int32_t* flatten_ids;
  int64_t N;
  int channels;
  int W, H, ts, tw, th;
  int64_t I;
  int64_t n_isects;
};

// Range of the tile's list; the last tile of the last image ends at n_isects
// (gsplat_rasterize.cpp:296-299).
__device__ __forceinline__ void tile_range(const RasterArgs& a, int64_t image, int tile, int64_t* start,
                                           int64_t* end) {
  const int64_t n_tiles = static_cast<int64_t>(a.tw) * a.th;
  const int64_t oi = image * n_tiles + tile;
  const int64_t s = a.tile_offsets[oi];
  const int64_t e = (oi + 1 == a.I * n_tiles) ? a.n_isects : a.tile_offsets[oi + 1];
  // consistent offsets already satisfy 0 <= s <= e <= n_isects; clamping only
  // keeps reads in bounds for inconsistent caller data
  *start = min(max<int64_t>(s, 0), a.n_isects);
  *end = min(max(e, *start), a.n_isects);
}

// Gaussian record of list entry j; ids outside [0, I*N) read as a
// zero-opacity Gaussian (never contributes) instead of reading out of bounds.
__device__ __forceinline__ int32_t load_gaussian(const RasterArgs& a, int64_t j, float2* xy, float4* co) {
  int32_t g = a.flatten_ids[j];
  if (g < 0 || static_cast<int64_t>(g) >= a.I * a.N) {
    *xy = make_float2(0.0f, 0.0f);
    *co = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    return 0;
  }
  const int64_t gg = g;
  *xy = make_float2(a.means2d[gg * 2], a.means2d[gg * 2 + 1]);
  *co = make_float4(a.conics[gg * 3], a.conics[gg * 3 + 1], a.conics[gg * 3 + 2], a.opacities[gg]);
  return g;
}

// CH in 1..4: colors staged in LDS; CH == 0: runtime channel count (<= 64),
// colors read from global memory.
template <int CH>
__global__ void __launch_bounds__(1024) raster_fwd_kernel(RasterArgs a, float* __restrict__ render_colors,
                                                          float* __restrict__ render_alphas,
                                                          int32_t* __restrict__ last_ids) {
  constexpr int LC = CH > 0 ? CH : 1;
  extern __shared__ float smem[];
  const int BS = blockDim.x;
  float2* s_xy = reinterpret_cast<float2*>(smem);
  float4* s_co = reinterpret_cast<float4*>(smem + 2 * BS);  // conic xyz, opacity
  float* s_col = smem + 6 * BS;                            // [BS][LC] (CH > 0)
  int32_t* s_g = reinterpret_cast<int32_t*>(smem + 6 * BS + (CH > 0 ? LC * BS : 0));

  const int channels = CH > 0 ? CH : a.channels;
  const int tx = blockIdx.x, ty = blockIdx.y;
  const int64_t image = blockIdx.z;
  const int tile = ty * a.tw + tx;
  const int t = threadIdx.x;
  const int x = tx * a.ts + t % a.ts;
  const int y = ty * a.ts + t / a.ts;
  // blocks are padded to whole wave64s; padding lanes own no pixel
  const bool inside = t < a.ts * a.ts && x < a.W && y < a.H;
  const int64_t pix = (image * a.H + y) * static_cast<int64_t>(a.W) + x;
  const float* bg = a.backgrounds ? a.backgrounds + image * channels : nullptr;
  const int64_t n_tiles = static_cast<int64_t>(a.tw) * a.th;

  if (a.masks && !a.masks[image * n_tiles + tile]) {
    if (inside) {
      render_alphas[pix] = 0.0f;
      for (int c = 0; c < channels; ++c) render_colors[pix * channels + c] = bg ? bg[c] : 0.0f;
      last_ids[pix] = 0;
    }
    return;
  }
  int64_t start, end;
  tile_range(a, image, tile, &start, &end);
  const float px = static_cast<float>(x) + 0.5f;
  const float py = static_cast<float>(y) + 0.5f;
  float T = 1.0f;
  int32_t cur = 0;
  float acc[CH > 0 ? CH : kMaxChannels];
#pragma unroll
  for (int c = 0; c < (CH > 0 ? CH : kMaxChannels); ++c) acc[c] = 0.0f;
  bool done = !inside;

  for (int64_t b0 = start; b0 < end; b0 += BS) {
    if (__syncthreads_count(done) == BS) break;  // also fences the previous batch's LDS reads
    const int64_t j = b0 + t;
    if (j < end) {
      float2 xy;
      float4 co;
      const int32_t g = load_gaussian(a, j, &xy, &co);
      s_xy[t] = xy;
      s_co[t] = co;
      if constexpr (CH > 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c) s_col[t * CH + c] = a.colors[static_cast<int64_t>(g) * CH + c];
      } else {
        s_g[t] = g;
      }
    }
    __syncthreads();
    const int cnt = static_cast<int>(min<int64_t>(BS, end - b0));
    if (!done) {
      for (int k = 0; k < cnt; ++k) {
        const float2 m = s_xy[k];
        const float4 co = s_co[k];
        const float dx = m.x - px;
        const float dy = m.y - py;
        const float sigma = 0.5f * (co.x * dx * dx + co.z * dy * dy) + co.y * dx * dy;
        const float alpha = fminf(kMaxAlpha, co.w * expf(-sigma));
        if (sigma < 0.0f || alpha < kAlphaThreshold) continue;
        const float next_T = T * (1.0f - alpha);
        if (next_T <= kTransmittanceThreshold) {
          done = true;
          break;
        }
        const float vis = alpha * T;
        if constexpr (CH > 0) {
#pragma unroll
          for (int c = 0; c < CH; ++c) acc[c] += s_col[k * CH + c] * vis;
        } else {
          const float* col = a.colors + static_cast<int64_t>(s_g[k]) * channels;
          for (int c = 0; c < channels; ++c) acc[c] += col[c] * vis;
        }
        cur = static_cast<int32_t>(b0 + k);
        T = next_T;
      }
    }
  }
  if (!inside) return;
  render_alphas[pix] = 1.0f - T;
  if constexpr (CH > 0) {
#pragma unroll
    for (int c = 0; c < CH; ++c) render_colors[pix * CH + c] = acc[c] + T * (bg ? bg[c] : 0.0f);
  } else {
    for (int c = 0; c < channels; ++c) render_colors[pix * channels + c] = acc[c] + T * (bg ? bg[c] : 0.0f);
  }
  last_ids[pix] = cur;
}

// Adds a wave-reduced value to *dst from one lane (dst is wave-uniform).
__device__ __forceinline__ void wave_atomic_add(float* dst, float v, int lane) {
  const float s = wave_sum_uniform(v);
  if (lane == 0) unsafeAtomicAdd(dst, s);
}

template <int CH>
__global__ void __launch_bounds__(1024) raster_bwd_kernel(RasterArgs a, const float* __restrict__ render_alphas,
                                                          const int32_t* __restrict__ last_ids,
                                                          const float* __restrict__ v_render_colors,
                                                          const float* __restrict__ v_render_alphas,
                                                          float* __restrict__ v_means2d_abs,
                                                          float* __restrict__ v_means2d, float* __restrict__ v_conics,
                                                          float* __restrict__ v_colors, float* __restrict__ v_opacities,
                                                          float* __restrict__ v_backgrounds) {
  constexpr int LC = CH > 0 ? CH : 1;
  constexpr int AC = CH > 0 ? CH : kMaxChannels;
  extern __shared__ float smem[];
  const int BS = blockDim.x;
  float2* s_xy = reinterpret_cast<float2*>(smem);
  float4* s_co = reinterpret_cast<float4*>(smem + 2 * BS);
  int32_t* s_g = reinterpret_cast<int32_t*>(smem + 6 * BS);
  float* s_col = smem + 7 * BS;  // [BS][LC] (CH > 0)
  __shared__ int s_max_last;

  const int channels = CH > 0 ? CH : a.channels;
  const int tx = blockIdx.x, ty = blockIdx.y;
  const int64_t image = blockIdx.z;
  const int tile = ty * a.tw + tx;
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int x = tx * a.ts + t % a.ts;
  const int y = ty * a.ts + t / a.ts;
  // blocks are padded to whole wave64s (the DPP reductions need every lane);
  // padding lanes own no pixel
  const bool inside = t < a.ts * a.ts && x < a.W && y < a.H;
  const int64_t pix = (image * a.H + y) * static_cast<int64_t>(a.W) + x;
  const int64_t n_tiles = static_cast<int64_t>(a.tw) * a.th;
  if (a.masks && !a.masks[image * n_tiles + tile]) return;  // masked tiles contribute nothing
  const float* bg = a.backgrounds ? a.backgrounds + image * channels : nullptr;

  int64_t start, end;
  tile_range(a, image, tile, &start, &end);
  const float px = static_cast<float>(x) + 0.5f;
  const float py = static_cast<float>(y) + 0.5f;
  const float T_final = inside ? 1.0f - render_alphas[pix] : 1.0f;
  float T = T_final;
  const int64_t bin_final = inside ? last_ids[pix] : -1;
  float v_rc[AC];
  float buffer[AC];
  float bg_dot = 0.0f;
  for (int c = 0; c < channels; ++c) {
    v_rc[c] = inside ? v_render_colors[pix * channels + c] : 0.0f;
    buffer[c] = 0.0f;
  }
  const float v_ra = inside ? v_render_alphas[pix] : 0.0f;
  if (bg) {
    for (int c = 0; c < channels; ++c) bg_dot += bg[c] * v_rc[c];
    // v_backgrounds = sum over pixels of T_final * v_rc (gsplat_rasterize.cpp:459-464)
    for (int c = 0; c < channels; ++c) wave_atomic_add(v_backgrounds + image * channels + c, T_final * v_rc[c], lane);
  }

  // Entries past every lane's last contributor are skipped wholesale.
  if (t == 0) s_max_last = -1;
  __syncthreads();
  const int64_t my_last = inside ? min<int64_t>(end - 1, bin_final) : start - 1;
  if (my_last >= start) atomicMax(&s_max_last, static_cast<int>(my_last - start));
  __syncthreads();
  const int64_t stop = start + s_max_last + 1;  // exclusive end of the needed range

  for (int64_t b1 = stop; b1 > start; b1 -= BS) {
    const int64_t b0 = max<int64_t>(start, b1 - BS);
    __syncthreads();  // previous batch fully consumed
    const int64_t j = b1 - 1 - t;  // slot k holds entry b1 - 1 - k (back to front)
    if (j >= b0) {
      float2 xy;
      float4 co;
      const int32_t g = load_gaussian(a, j, &xy, &co);
      s_xy[t] = xy;
      s_co[t] = co;
      s_g[t] = g;
      if constexpr (CH > 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c) s_col[t * CH + c] = a.colors[static_cast<int64_t>(g) * CH + c];
      }
    }
    __syncthreads();
    const int cnt = static_cast<int>(b1 - b0);
    for (int k = 0; k < cnt; ++k) {
      const int64_t idx = b1 - 1 - k;
      const float2 m = s_xy[k];
      const float4 co = s_co[k];
      const int32_t g = s_g[k];
      const float dx = m.x - px;
      const float dy = m.y - py;
      const float sigma = 0.5f * (co.x * dx * dx + co.z * dy * dy) + co.y * dx * dy;
      const float vis = expf(-sigma);
      const float alpha = fminf(kMaxAlpha, co.w * vis);
      const bool valid = idx <= bin_final && !(sigma < 0.0f || alpha < kAlphaThreshold);
      if (__ballot(valid) == 0) continue;
      float v_col[AC];
      float v_c0 = 0.0f, v_c1 = 0.0f, v_c2 = 0.0f, v_x = 0.0f, v_y = 0.0f, v_op = 0.0f;
      for (int c = 0; c < channels; ++c) v_col[c] = 0.0f;
      if (valid) {
        const float ra = 1.0f / fmaxf(kMinOneMinusAlpha, 1.0f - alpha);
        T *= ra;
        const float fac = alpha * T;
        float v_alpha = 0.0f;
        if constexpr (CH > 0) {
#pragma unroll
          for (int c = 0; c < CH; ++c) {
            v_col[c] = fac * v_rc[c];
            v_alpha += (s_col[k * CH + c] * T - buffer[c] * ra) * v_rc[c];
          }
        } else {
          const float* col = a.colors + static_cast<int64_t>(g) * channels;
          for (int c = 0; c < channels; ++c) {
            v_col[c] = fac * v_rc[c];
            v_alpha += (col[c] * T - buffer[c] * ra) * v_rc[c];
          }
        }
        v_alpha += T_final * ra * v_ra;
        if (bg) v_alpha += -T_final * ra * bg_dot;
        if (co.w * vis <= kMaxAlpha) {
          const float v_sigma = -co.w * vis * v_alpha;
          v_x = v_sigma * (co.x * dx + co.y * dy);
          v_y = v_sigma * (co.y * dx + co.z * dy);
          v_c0 = 0.5f * v_sigma * dx * dx;
          v_c1 = v_sigma * dx * dy;
          v_c2 = 0.5f * v_sigma * dy * dy;
          v_op = vis * v_alpha;
        }
        if constexpr (CH > 0) {
#pragma unroll
          for (int c = 0; c < CH; ++c) buffer[c] += s_col[k * CH + c] * fac;
        } else {
          const float* col = a.colors + static_cast<int64_t>(g) * channels;
          for (int c = 0; c < channels; ++c) buffer[c] += col[c] * fac;
        }
      }
      const int64_t gg = g;
      for (int c = 0; c < channels; ++c) wave_atomic_add(v_colors + gg * channels + c, v_col[c], lane);
      wave_atomic_add(v_conics + gg * 3, v_c0, lane);
      wave_atomic_add(v_conics + gg * 3 + 1, v_c1, lane);
      wave_atomic_add(v_conics + gg * 3 + 2, v_c2, lane);
      wave_atomic_add(v_means2d + gg * 2, v_x, lane);
      wave_atomic_add(v_means2d + gg * 2 + 1, v_y, lane);
      wave_atomic_add(v_opacities + gg, v_op, lane);
      if (v_means2d_abs) {
        wave_atomic_add(v_means2d_abs + gg * 2, fabsf(v_x), lane);
        wave_atomic_add(v_means2d_abs + gg * 2 + 1, fabsf(v_y), lane);
      }
    }
  }
}

size_t fwd_smem(int ch, int bs) { return static_cast<size_t>(bs) * (6 + (ch > 0 ? ch : 0) + (ch > 0 ? 0 : 1)) * 4; }
size_t bwd_smem(int ch, int bs) { return static_cast<size_t>(bs) * (7 + (ch > 0 ? ch : 0)) * 4; }

int check_args(const RasterArgs& a, const char* what) {
  if (a.I < 0 || a.N < 0 || a.channels <= 0 || a.W < 0 || a.H < 0 || a.ts <= 0 || a.tw < 0 || a.th < 0 ||
      a.n_isects < 0)
    return invalid(std::string(what) + ": invalid sizes.");
  if (a.channels > kMaxChannels)
    return invalid(std::string(what) + ": at most 64 channels are supported.");
  if (a.ts * a.ts > 1024) return invalid(std::string(what) + ": tile_size must be at most 32.");
  if (static_cast<int64_t>(a.tw) * a.ts < a.W || static_cast<int64_t>(a.th) * a.ts < a.H)
    return invalid(std::string(what) + ": tile grid does not cover the image.");
  if (a.I > 65535 || a.th > 65535) return invalid(std::string(what) + ": too many images or tile rows.");
  return GSPLAT_OK;
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" int gsplat_hip_rasterize_fwd(const float* means2d, const float* conics, const float* colors,
                                        const float* opacities, const float* backgrounds, const uint8_t* masks,
                                        const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I, int64_t N,
                                        int32_t channels, int32_t image_width, int32_t image_height, int32_t tile_size,
                                        int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                        float* render_colors, float* render_alphas, int32_t* last_ids, void* stream) {
  RasterArgs a{means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, N, channels,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects};
  int rc = check_args(a, "rasterize_to_pixels_3dgs_forward");
  if (rc) return rc;
  if (I == 0 || tile_width == 0 || tile_height == 0) return GSPLAT_OK;
  if (!tile_offsets || !render_colors || !render_alphas || !last_ids || (n_isects > 0 && !flatten_ids))
    return invalid("rasterize_to_pixels_3dgs_forward: null pointer.");
  if (n_isects > 0 && (!means2d || !conics || !colors || !opacities))
    return invalid("rasterize_to_pixels_3dgs_forward: null pointer.");
  const dim3 grid(tile_width, tile_height, static_cast<unsigned>(I));
  const int bs = (tile_size * tile_size + kWave - 1) / kWave * kWave;
  hipStream_t s = as_stream(stream);
  const int ch = channels <= 4 ? channels : 0;
  const size_t sm = fwd_smem(ch, bs);
  switch (ch) {
    case 1: raster_fwd_kernel<1><<<grid, bs, sm, s>>>(a, render_colors, render_alphas, last_ids); break;
    case 2: raster_fwd_kernel<2><<<grid, bs, sm, s>>>(a, render_colors, render_alphas, last_ids); break;
    case 3: raster_fwd_kernel<3><<<grid, bs, sm, s>>>(a, render_colors, render_alphas, last_ids); break;
    case 4: raster_fwd_kernel<4><<<grid, bs, sm, s>>>(a, render_colors, render_alphas, last_ids); break;
    default: raster_fwd_kernel<0><<<grid, bs, sm, s>>>(a, render_colors, render_alphas, last_ids); break;
  }
  return check_launch("rasterize_to_pixels_3dgs_forward");
}

extern "C" int gsplat_hip_rasterize_bwd(const float* means2d, const float* conics, const float* colors,
                                        const float* opacities, const float* backgrounds, const uint8_t* masks,
                                        const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I, int64_t N,
                                        int32_t channels, int32_t image_width, int32_t image_height, int32_t tile_size,
                                        int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                        const float* render_alphas, const int32_t* last_ids,
                                        const float* v_render_colors, const float* v_render_alphas,
                                        float* v_means2d_abs, float* v_means2d, float* v_conics, float* v_colors,
                                        float* v_opacities, float* v_backgrounds, void* stream) {
  RasterArgs a{means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, N, channels,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects};
  int rc = check_args(a, "rasterize_to_pixels_3dgs_backward");
  if (rc) return rc;
  if (!v_means2d || !v_conics || !v_colors || !v_opacities)
    return invalid("rasterize_to_pixels_3dgs_backward: null pointer.");
  if (backgrounds && !v_backgrounds) return invalid("rasterize_to_pixels_3dgs_backward: null v_backgrounds.");
  hipStream_t s = as_stream(stream);
  const int64_t G = I * N;
  // outputs are accumulated: clear them first
  if ((rc = fill_zero(v_means2d, G * 2 * sizeof(float), s))) return rc;
  if ((rc = fill_zero(v_conics, G * 3 * sizeof(float), s))) return rc;
  if ((rc = fill_zero(v_colors, G * channels * sizeof(float), s))) return rc;
  if ((rc = fill_zero(v_opacities, G * sizeof(float), s))) return rc;
  if (v_means2d_abs && (rc = fill_zero(v_means2d_abs, G * 2 * sizeof(float), s))) return rc;
  if (backgrounds && (rc = fill_zero(v_backgrounds, I * channels * sizeof(float), s))) return rc;
  if (I == 0 || tile_width == 0 || tile_height == 0) return GSPLAT_OK;
  if (!tile_offsets || !render_alphas || !last_ids || !v_render_colors || !v_render_alphas ||
      (n_isects > 0 && (!flatten_ids || !means2d || !conics || !colors || !opacities)))
    return invalid("rasterize_to_pixels_3dgs_backward: null pointer.");
  const dim3 grid(tile_width, tile_height, static_cast<unsigned>(I));
  const int bs = (tile_size * tile_size + kWave - 1) / kWave * kWave;
  const int ch = channels <= 4 ? channels : 0;
  const size_t sm = bwd_smem(ch, bs);
#define GSPLAT_BWD_LAUNCH(C)                                                                                     \
  raster_bwd_kernel<C><<<grid, bs, sm, s>>>(a, render_alphas, last_ids, v_render_colors, v_render_alphas,        \
                                            v_means2d_abs, v_means2d, v_conics, v_colors, v_opacities,           \
                                            v_backgrounds)
  switch (ch) {
    case 1: GSPLAT_BWD_LAUNCH(1); break;
    case 2: GSPLAT_BWD_LAUNCH(2); break;
    case 3: GSPLAT_BWD_LAUNCH(3); break;
    case 4: GSPLAT_BWD_LAUNCH(4); break;
    default: GSPLAT_BWD_LAUNCH(0); break;
  }
#undef GSPLAT_BWD_LAUNCH
  return check_launch("rasterize_to_pixels_3dgs_backward");
}
