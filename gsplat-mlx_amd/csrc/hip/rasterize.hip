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

// Wave-wide sums of NV values, interleaved so the independent DPP chains hide
// each other's hazards: row_shr 1/2/4/8 within each 16-lane row, then
// row_bcast 15 / 31 across rows; lane 63 ends up with the wave total.
template <int NV>
__device__ __forceinline__ void wave_reduce_lane63(float (&v)[NV]) {
#pragma unroll
  for (int step = 0; step < 6; ++step) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int x = __builtin_bit_cast(int, v[i]);
      int y;
      switch (step) {
        case 0: y = __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false); break;  // row_shr:1
        case 1: y = __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false); break;  // row_shr:2
        case 2: y = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false); break;  // row_shr:4
        case 3: y = __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false); break;  // row_shr:8
        case 4: y = __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false); break;  // row_bcast:15
        default: y = __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false); break; // row_bcast:31
      }
      v[i] += __builtin_bit_cast(float, y);
    }
  }
}

// Backward. The tile's list is walked back-to-front in batches of BB entries
// from the block's largest last_id. For each entry every lane computes its
// pixel's partial gradients; a wave with at least one contributing lane sums
// them across the wave (DPP) and lane 63 stores the NV sums into the wave's
// own accumulator slot for that entry (plain LDS stores: each (wave, entry)
// slot is written at most once per batch, so no LDS atomics). After the batch
// the block adds up the per-wave slots and flushes one global atomic per
// (entry, nonzero component).
template <int CH, bool ABS>
__global__ void __launch_bounds__(1024) raster_bwd_kernel(RasterArgs a, int BB, const float* __restrict__ render_alphas,
                                                          const int32_t* __restrict__ last_ids,
                                                          const float* __restrict__ v_render_colors,
                                                          const float* __restrict__ v_render_alphas,
                                                          float* __restrict__ v_means2d_abs,
                                                          float* __restrict__ v_means2d, float* __restrict__ v_conics,
                                                          float* __restrict__ v_colors, float* __restrict__ v_opacities,
                                                          float* __restrict__ v_backgrounds) {
  constexpr int LC = CH > 0 ? CH : 1;
  constexpr int AC = CH > 0 ? CH : kMaxChannels;
  // accumulated components per Gaussian: colors (CH), conic (3), mean (2),
  // opacity (1), |mean| (2, absgrad only)
  constexpr int NG = ABS ? 8 : 6;  // geometry components
  constexpr int NV = (CH > 0 ? CH : 0) + NG;
  extern __shared__ float smem[];
  const int BS = blockDim.x;
  const int n_waves = BS / kWave;
  float2* s_xy = reinterpret_cast<float2*>(smem);            // [BB]
  float4* s_co = reinterpret_cast<float4*>(smem + 2 * BB);   // [BB] conic xyz, opacity
  int32_t* s_g = reinterpret_cast<int32_t*>(smem + 6 * BB);  // [BB]
  float* s_col = smem + 7 * BB;                              // [BB][LC] (CH > 0)
  float* s_acc = s_col + (CH > 0 ? LC * BB : 0);             // [n_waves][BB][NV]
  __shared__ int s_max_last;

  const int channels = CH > 0 ? CH : a.channels;
  const int tx = blockIdx.x, ty = blockIdx.y;
  const int64_t image = blockIdx.z;
  const int tile = ty * a.tw + tx;
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
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
    for (int c = 0; c < channels; ++c) {
      const float s = wave_sum_uniform(T_final * v_rc[c]);
      if (lane == 0) unsafeAtomicAdd(v_backgrounds + image * channels + c, s);
    }
  }
  const float t_final_ra_coef = T_final * v_ra;  // times ra below
  const float t_final_bg_coef = -T_final * bg_dot;

  // Entries past every lane's last contributor are skipped wholesale: the
  // block starts at its largest last_id, each wave skips entries past its own.
  if (t == 0) s_max_last = -1;
  __syncthreads();
  const int64_t my_last = inside ? min<int64_t>(end - 1, bin_final) : start - 1;
  if (my_last >= start) atomicMax(&s_max_last, static_cast<int>(my_last - start));
  int64_t wave_last = my_last;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) wave_last = max(wave_last, __shfl_xor(wave_last, off, kWave));
  __syncthreads();
  const int64_t stop = start + s_max_last + 1;  // exclusive end of the needed range
  const int acc_words = n_waves * BB * NV;

  for (int64_t b1 = stop; b1 > start; b1 -= BB) {
    const int64_t b0 = max<int64_t>(start, b1 - BB);
    __syncthreads();  // previous batch fully consumed and flushed
    const int64_t j = b1 - 1 - t;  // slot k holds entry b1 - 1 - k (back to front)
    if (t < BB && j >= b0) {
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
    // acc_words is a multiple of 4 (BB is a multiple of 64)
    for (int w = t * 4; w < acc_words; w += BS * 4)
      *reinterpret_cast<float4*>(s_acc + w) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    __syncthreads();
    const int cnt = static_cast<int>(b1 - b0);
    for (int k = 0; k < cnt; ++k) {
      const int64_t idx = b1 - 1 - k;
      if (idx > wave_last) continue;  // wave-uniform
      const float2 m = s_xy[k];
      const float4 co = s_co[k];
      const float dx = m.x - px;
      const float dy = m.y - py;
      const float sigma = 0.5f * (co.x * dx * dx + co.z * dy * dy) + co.y * dx * dy;
      const float vis = expf(-sigma);
      const float alpha = fminf(kMaxAlpha, co.w * vis);
      const bool valid = idx <= bin_final && !(sigma < 0.0f || alpha < kAlphaThreshold);
      if (__ballot(valid) == 0) continue;
      float v[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) v[i] = 0.0f;
      float v_col_generic[CH > 0 ? 1 : kMaxChannels];
      if (valid) {
        const float ra = __builtin_amdgcn_rcpf(fmaxf(kMinOneMinusAlpha, 1.0f - alpha));
        T *= ra;
        const float fac = alpha * T;
        float v_alpha = 0.0f;
        if constexpr (CH > 0) {
#pragma unroll
          for (int c = 0; c < CH; ++c) {
            const float col = s_col[k * CH + c];
            v[c] = fac * v_rc[c];
            v_alpha += (col * T - buffer[c] * ra) * v_rc[c];
            buffer[c] += col * fac;
          }
        } else {
          const float* col = a.colors + static_cast<int64_t>(s_g[k]) * channels;
          for (int c = 0; c < channels; ++c) {
            v_col_generic[c] = fac * v_rc[c];
            v_alpha += (col[c] * T - buffer[c] * ra) * v_rc[c];
            buffer[c] += col[c] * fac;
          }
        }
        v_alpha += ra * (t_final_ra_coef + t_final_bg_coef);
        if (co.w * vis <= kMaxAlpha) {
          const float v_sigma = -co.w * vis * v_alpha;
          const float vx = v_sigma * (co.x * dx + co.y * dy);
          const float vy = v_sigma * (co.y * dx + co.z * dy);
          constexpr int o = CH > 0 ? CH : 0;
          v[o + 0] = 0.5f * v_sigma * dx * dx;
          v[o + 1] = v_sigma * dx * dy;
          v[o + 2] = 0.5f * v_sigma * dy * dy;
          v[o + 3] = vx;
          v[o + 4] = vy;
          v[o + 5] = vis * v_alpha;
          if constexpr (ABS) {
            v[o + 6] = fabsf(vx);
            v[o + 7] = fabsf(vy);
          }
        }
      } else if constexpr (CH == 0) {
        for (int c = 0; c < channels; ++c) v_col_generic[c] = 0.0f;
      }
      if constexpr (CH == 0) {
        // generic channel count: colour gradients go straight to global memory
        const int64_t gg = s_g[k];
        for (int c = 0; c < channels; ++c) {
          const float s = wave_sum_uniform(v_col_generic[c]);
          if (lane == 0 && s != 0.0f) unsafeAtomicAdd(v_colors + gg * channels + c, s);
        }
      }
      wave_reduce_lane63<NV>(v);
      if (lane == kWave - 1) {
        float* acc = s_acc + (wave * BB + k) * NV;
#pragma unroll
        for (int i = 0; i < NV; ++i) acc[i] = v[i];
      }
    }
    __syncthreads();
    // flush: thread t owns slot t (entry b1 - 1 - t); sums the waves' slots
    if (t < cnt) {
      float acc[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) acc[i] = s_acc[t * NV + i];
      for (int w = 1; w < n_waves; ++w) {
#pragma unroll
        for (int i = 0; i < NV; ++i) acc[i] += s_acc[(w * BB + t) * NV + i];
      }
      const int64_t gg = s_g[t];
      constexpr int o = CH > 0 ? CH : 0;
      if constexpr (CH > 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
          if (acc[c] != 0.0f) unsafeAtomicAdd(v_colors + gg * CH + c, acc[c]);
      }
      if (acc[o + 0] != 0.0f) unsafeAtomicAdd(v_conics + gg * 3, acc[o + 0]);
      if (acc[o + 1] != 0.0f) unsafeAtomicAdd(v_conics + gg * 3 + 1, acc[o + 1]);
      if (acc[o + 2] != 0.0f) unsafeAtomicAdd(v_conics + gg * 3 + 2, acc[o + 2]);
      if (acc[o + 3] != 0.0f) unsafeAtomicAdd(v_means2d + gg * 2, acc[o + 3]);
      if (acc[o + 4] != 0.0f) unsafeAtomicAdd(v_means2d + gg * 2 + 1, acc[o + 4]);
      if (acc[o + 5] != 0.0f) unsafeAtomicAdd(v_opacities + gg, acc[o + 5]);
      if constexpr (ABS) {
        if (acc[o + 6] != 0.0f) unsafeAtomicAdd(v_means2d_abs + gg * 2, acc[o + 6]);
        if (acc[o + 7] != 0.0f) unsafeAtomicAdd(v_means2d_abs + gg * 2 + 1, acc[o + 7]);
      }
    }
  }
}

size_t fwd_smem(int ch, int bs) { return static_cast<size_t>(bs) * (6 + (ch > 0 ? ch : 0) + (ch > 0 ? 0 : 1)) * 4; }
// Backward batch length: 128 entries for blocks of up to 256 lanes, 64 above
// (bounds the per-wave accumulators to 48 KiB at 1024 lanes, 4 channels,
// absgrad); never more than the block so one lane loads one record.
int bwd_batch(int bs) { return bs <= 128 ? bs : (bs <= 256 ? 128 : 64); }
// records (7 + colors) per batch slot plus NV accumulators per (wave, slot)
size_t bwd_smem(int ch, int bs, bool absgrad) {
  const int bb = bwd_batch(bs);
  const int cc = ch > 0 ? ch : 0;
  const int nv = cc + (absgrad ? 8 : 6);
  return static_cast<size_t>(bb) * (7 + cc + (bs / kWave) * nv) * 4;
}

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
  KernelTimer timer("raster_fwd", s);
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
  const size_t sm = bwd_smem(ch, bs, v_means2d_abs != nullptr);
  const int bb = bwd_batch(bs);
  KernelTimer timer("raster_bwd", s);
#define GSPLAT_BWD_LAUNCH(C)                                                                                     \
  if (v_means2d_abs)                                                                                             \
    raster_bwd_kernel<C, true><<<grid, bs, sm, s>>>(a, bb, render_alphas, last_ids, v_render_colors, v_render_alphas, \
                                                    v_means2d_abs, v_means2d, v_conics, v_colors, v_opacities,   \
                                                    v_backgrounds);                                              \
  else                                                                                                           \
    raster_bwd_kernel<C, false><<<grid, bs, sm, s>>>(a, bb, render_alphas, last_ids, v_render_colors,                 \
                                                     v_render_alphas, nullptr, v_means2d, v_conics, v_colors,     \
                                                     v_opacities, v_backgrounds)
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
