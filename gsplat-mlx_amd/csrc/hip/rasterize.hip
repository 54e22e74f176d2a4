// Tile rasterization (front-to-back alpha compositing) forward / backward for
// gfx950.
//
// Forward: one block per (image, tile) with tile_size^2 lanes, one pixel per
// lane (16x16 tiles -> 4 wave64s, each covering an 8x8 block). The tile's
// sorted Gaussian list is walked in batches of blockDim entries: each lane
// gathers one Gaussian record (mean, conic, opacity, colors) into LDS and
// tests it against every wave's pixel rectangle, then each wave evaluates
// only the records that may touch it. The forward stops when every lane of
// the block has saturated (block vote).
//
// Backward: one block per tile, dispatched heaviest tile first, replays the
// tile's list back-to-front from its largest last_id, rebuilding
// transmittance per pixel; per record, a wave sums its lanes' partial
// gradients by a transposed DPP/permlane reduction into per-wave LDS slots,
// and each batch ends with one atomic per (record, nonzero component).
//
// Per-pixel math follows gsplat_core/gsplat_rasterize.cpp:291-368 (forward)
// and :432-554 (backward) operation for operation; the Gaussian falloff and
// alpha tests are evaluated exactly as the reference (no FMA contraction in
// this file; the backward's gradient arithmetic uses explicit FMAs) so
// compositing decisions match it.
#include <algorithm>
#include <atomic>
#include <climits>
#include <mutex>

#include "common.hpp"
#include "scan.hpp"

// Scratch of gsplat_hip_rasterize_bwd_noalloc: the backward's tile schedule
// (cost and order per tile) and background-gradient partials (per tile and
// channel), in device memory that every GPU the library runs on holds from
// load to process end. Host code never uses this name as an address: the
// address is looked up per device (noalloc_scratch below).
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(8) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace gsplat_hip {
namespace {

constexpr int kMaxChannels = 64;

// Words of one backward batch record in LDS: conic xyz + opacity, then mean
// xy, the CH staged colours (none for CH == 0), the Gaussian id and the
// per-wave touch mask, padded to 16 bytes.
__host__ __device__ constexpr int bwd_record_words(int ch) { return 4 + (2 + ch + 2 + 3) / 4 * 4; }

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
  int64_t G;  // Gaussian rows: I * N (dense) or nnz (packed)
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

// Gaussian record of list entry j; ids outside [0, G) read as a
// zero-opacity Gaussian (never contributes) instead of reading out of bounds.
__device__ __forceinline__ int32_t load_gaussian(const RasterArgs& a, int64_t j, float2* xy, float4* co) {
  int32_t g = a.flatten_ids[j];
  if (g < 0 || static_cast<int64_t>(g) >= a.G) {
    *xy = make_float2(0.0f, 0.0f);
    *co = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    return 0;
  }
  const int64_t gg = g;
  *xy = make_float2(a.means2d[gg * 2], a.means2d[gg * 2 + 1]);
  *co = make_float4(a.conics[gg * 3], a.conics[gg * 3 + 1], a.conics[gg * 3 + 2], a.opacities[gg]);
  return g;
}

// exp(y) by Cody-Waite reduction: y log2(e) = n + f with the product kept
// exact to about 2^-48 (log2(e) split into a float head and tail, the head's
// rounding error recovered by an FMA), 2^f from v_exp_f32, scaled by 2^n.
// The tail is log2(e) - head truncated to float (0x32a5705f), the value the
// device library's expf uses, which makes this bit-identical to expf for
// every float y > -103 (compared exhaustively on gfx950); it only drops
// expf's range selects.
//
// Below -104 the argument is raised to -104 first (IEEE maximum: one
// v_maximum3_f32, NaN passes through). Without it the reduction breaks down
// for y < -2.98e9, where ulp(y log2 e) >= 256 leaves a residual f >= 128 and
// 2^f overflows (ldexp(inf, n) = inf), and for y = -inf, where the head's
// error term is inf - inf = NaN. With it every y <= -104 gives at most
// 2^-149, so o * exp fails the 1/255 alpha test for any finite opacity, as
// expf's 0 does; a NaN argument still yields NaN (alpha = min(0.99, NaN) =
// 0.99, the reference's std::min result).
__device__ __forceinline__ float exp_alpha(float y) {
  const float head = 1.44269502162933349609375f;  // float(log2 e)
  const float tail = __uint_as_float(0x32a5705fu);
  y = __builtin_elementwise_maximum(y, -104.0f);
  const float ph = y * head;
  float pl = __builtin_fmaf(y, head, -ph);
  pl = __builtin_fmaf(y, tail, pl);
  const float n = __builtin_rintf(ph);
  const float f = (ph - n) + pl;
  return __builtin_ldexpf(__builtin_amdgcn_exp2f(f), static_cast<int>(n));
}

// ---------------------------------------------------------------------------
// Per-wave culling. When a batch record is staged, its loader tests it once
// against every wave's pixel rectangle and stores a bit mask; each wave
// collects the set bits of 64 records at a time with one ballot and visits
// only those records. A bit is cleared only when no pixel of the wave can
// pass the alpha test: alpha = min(0.99, o exp(-sigma)) >= 1/255 needs
// sigma <= ln(255 o), and the minimum of sigma over the rectangle of the
// wave's pixel centres (a positive-definite quadratic: zero if the mean is
// inside, else the smallest of the four clamped edge minima) exceeds
// 1.05 ln(255 o) + 1e-4. For conics with det > 1e-4 c0 c2 the float32
// rounding of that minimum and of the per-pixel sigma, exp and threshold is
// below 1%, well inside the slack; other conics, non-finite values and NaN
// opacities are never culled, and opacities <= 0 always are (alpha <= 0).
// Culled records cannot change a pixel of that wave, so results are
// unchanged.
struct PixRect {
  float x0, x1, y0, y1;
};

// Lane -> pixel of a tile. When the tile side is a multiple of 8, each
// wave64 owns an 8x8 block (waves row-major over the blocks); the square
// footprint is touched by fewer Gaussians than a 16x4 strip of the same
// area, so fewer records pass the per-wave cull. Other tile sides map lanes
// row-major. Lanes past ts*ts (padding) map outside the tile.
__device__ __forceinline__ void lane_pixel(int t, int ts, int* qx, int* qy) {
  if ((ts & 7) == 0) {
    const int w = t / kWave, l = t % kWave;
    const int bpr = ts >> 3;  // 8x8 blocks per tile row
    *qx = (w % bpr) * 8 + (l & 7);
    *qy = (w / bpr) * 8 + (l >> 3);
  } else {
    *qx = t % ts;
    *qy = t / ts;
  }
}

// Bounding rectangle of the pixel centres owned by wave w (lane_pixel's map).
__device__ __forceinline__ PixRect wave_rect(int w, int ts, int tx, int ty) {
  int c0, c1, r0, r1;
  if ((ts & 7) == 0) {
    const int bpr = ts >> 3;
    c0 = (w % bpr) * 8;
    c1 = c0 + 7;
    r0 = (w / bpr) * 8;
    r1 = r0 + 7;
  } else {
    const int q0 = w * kWave;
    const int q1 = min(q0 + kWave, ts * ts) - 1;
    r0 = q0 / ts;
    r1 = q1 / ts;
    c0 = 0;
    c1 = ts - 1;
    if (r0 == r1) {
      c0 = q0 % ts;
      c1 = q1 % ts;
    }
  }
  PixRect r;
  r.x0 = static_cast<float>(tx * ts + c0) + 0.5f;
  r.x1 = static_cast<float>(tx * ts + c1) + 0.5f;
  r.y0 = static_cast<float>(ty * ts + r0) + 0.5f;
  r.y1 = static_cast<float>(ty * ts + r1) + 0.5f;
  return r;
}

__device__ __forceinline__ float quad_form(float c0, float c1, float c2, float dx, float dy) {
  return 0.5f * (c0 * dx * dx + c2 * dy * dy) + c1 * dx * dy;
}

// A record's cull constants, formed once for all the rectangles it is tested
// against: the bound 1.05 ln(255 o) + 1e-4 on the minimum of sigma, and the
// conic's reciprocal diagonal for the clamped edge minimisers. Both come from
// the hardware approximations (v_log_f32, v_rcp_f32: about 1 ulp), far inside
// the slack; a denormal 255 o that v_log_f32 flushes gives ln = -inf, which
// culls the record as the exact logarithm (about -90) does. `always`: never
// culled (ill-conditioned or non-finite values, NaN opacity); `never`: always
// culled (opacity <= 0).
struct CullRec {
  float mx, my, c0, c1, c2, ic0, ic2, bound;
  bool always, never;
};

__device__ __forceinline__ CullRec cull_rec(float2 m, float4 co) {
  CullRec r;
  r.mx = m.x;
  r.my = m.y;
  r.c0 = co.x;
  r.c1 = co.y;
  r.c2 = co.z;
  const float o = co.w;
  r.never = o <= 0.0f;
  const float t = __builtin_amdgcn_logf(255.0f * o) * 0.69314718055994531f;  // log2 -> ln
  r.always = !r.never && (!(t < 1.0e30f) || !(r.c0 > 0.0f && r.c2 > 0.0f && r.c0 < 1.0e30f && r.c2 < 1.0e30f) ||
                          !(r.c0 * r.c2 - r.c1 * r.c1 > 1.0e-4f * r.c0 * r.c2) || !(fabsf(m.x) < 1.0e30f) ||
                          !(fabsf(m.y) < 1.0e30f));
  r.ic0 = __builtin_amdgcn_rcpf(r.c0);
  r.ic2 = __builtin_amdgcn_rcpf(r.c2);
  r.bound = 1.05f * t + 1.0e-4f;
  return r;
}

__device__ __forceinline__ bool may_touch(const CullRec& c, const PixRect& r) {
  if (c.never) return false;
  if (c.always) return true;
  if (c.mx >= r.x0 && c.mx <= r.x1 && c.my >= r.y0 && c.my <= r.y1) return true;
  float best = __builtin_huge_valf();
  // vertical edges (dx fixed), then horizontal edges (dy fixed)
  for (int e = 0; e < 2; ++e) {
    const float dx = c.mx - (e ? r.x1 : r.x0);
    const float dy = fminf(fmaxf(-c.c1 * dx * c.ic2, c.my - r.y1), c.my - r.y0);
    best = fminf(best, quad_form(c.c0, c.c1, c.c2, dx, dy));
  }
  for (int e = 0; e < 2; ++e) {
    const float dy = c.my - (e ? r.y1 : r.y0);
    const float dx = fminf(fmaxf(-c.c1 * dy * c.ic0, c.mx - r.x1), c.mx - r.x0);
    best = fminf(best, quad_form(c.c0, c.c1, c.c2, dx, dy));
  }
  return !(best > c.bound);
}

// The block's wave rectangles (x0, x1, y0, y1 per wave), formed once per
// block into LDS so that the staging lanes read them instead of converting
// the integer bounds for every record; visible after the block's next
// barrier.
__device__ __forceinline__ void store_wave_rects(float4* s_rect, int n_waves, int ts, int tx, int ty) {
  const int w = threadIdx.x;
  if (w < n_waves) {
    const PixRect r = wave_rect(w, ts, tx, ty);
    s_rect[w] = make_float4(r.x0, r.x1, r.y0, r.y1);
  }
}

__device__ __forceinline__ uint32_t touch_mask(float2 m, float4 co, int n_waves, const float4* s_rect) {
  const CullRec c = cull_rec(m, co);
  uint32_t mask = 0;
  for (int w = 0; w < n_waves; ++w) {
    const float4 r = s_rect[w];
    if (may_touch(c, PixRect{r.x, r.y, r.z, r.w})) mask |= 1u << w;
  }
  return mask;
}

// Words of one forward batch record in LDS: conic xyz + opacity, then mean xy
// and the CH staged colours (CH == 0: the Gaussian id), padded to 16 bytes.
__host__ __device__ constexpr int fwd_record_words(int ch) { return 4 + (2 + (ch > 0 ? ch : 1) + 3) / 4 * 4; }
// Touch-mask bit of a backward record whose mean or staged colours are not
// all finite.
constexpr uint32_t kNonFiniteRecord = 1u << 31;

// CH in 1..4: colors staged in LDS; CH == 0: runtime channel count (<= 64),
// colors read from global memory.
//
// Records are visited in pairs (the two falloffs and alpha tests are
// straight-line code that overlaps; compositing stays in list order, an odd
// count ends with an inert second visit). Each composite is an exec-masked
// branch taken by the lanes that keep the record.
template <int CH>
__global__ void __launch_bounds__(1024) raster_fwd_kernel(RasterArgs a, float* __restrict__ render_colors,
                                                          float* __restrict__ render_alphas,
                                                          int32_t* __restrict__ last_ids) {
  constexpr int FW = fwd_record_words(CH);
  extern __shared__ float smem[];
  const int BS = blockDim.x;
  float* s_rec = smem;                                               // [BS][FW]
  uint32_t* s_mask = reinterpret_cast<uint32_t*>(smem + FW * BS);   // [BS] per-wave touch bits
  float4* s_rect = reinterpret_cast<float4*>(smem + (FW + 1) * BS);  // [n_waves] wave pixel rects

  const int channels = CH > 0 ? CH : a.channels;
  const int tx = blockIdx.x, ty = blockIdx.y;
  const int64_t image = blockIdx.z;
  const int tile = ty * a.tw + tx;
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int n_waves = BS / kWave;
  int qx, qy;
  lane_pixel(t, a.ts, &qx, &qy);
  const int x = tx * a.ts + qx;
  const int y = ty * a.ts + qy;
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
  store_wave_rects(s_rect, n_waves, a.ts, tx, ty);
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
      float* rec = s_rec + t * FW;
      // conic diagonal pre-halved: (0.5 c0 dx) dx + (0.5 c2 dy) dy equals
      // 0.5 ((c0 dx) dx + (c2 dy) dy) bit for bit (scaling by 2 commutes with
      // rounding away from the subnormal range), one multiply less per visit
      *reinterpret_cast<float4*>(rec) = make_float4(0.5f * co.x, co.y, 0.5f * co.z, co.w);
      float tail[FW - 4];
#pragma unroll
      for (int i = 0; i < FW - 4; ++i) tail[i] = 0.0f;
      tail[0] = xy.x;
      tail[1] = xy.y;
      const uint32_t mask = touch_mask(xy, co, n_waves, s_rect);
      if constexpr (CH > 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c) tail[2 + c] = a.colors[static_cast<int64_t>(g) * CH + c];
      } else {
        tail[2] = __int_as_float(g);
      }
#pragma unroll
      for (int i = 0; i < FW - 4; i += 4)
        *reinterpret_cast<float4*>(rec + 4 + i) = make_float4(tail[i], tail[i + 1], tail[i + 2], tail[i + 3]);
      s_mask[t] = mask;
    }
    __syncthreads();
    const int cnt = static_cast<int>(min<int64_t>(BS, end - b0));

    // Compositing of one visit after its falloff (list order): skip when
    // sigma < 0 or alpha < 1/255; stop (without this record) when T would
    // fall to the threshold. The update is a branch, so the lanes that do not
    // take the record run it with their exec bit clear: they add nothing,
    // not even a non-finite colour, and a record no lane takes costs no
    // update at all.
    auto composite = [&](int k, const float4& xc, const float4& ex, bool pass_in, float alpha) {
      const bool pass = !done && pass_in;
      const float next_T = T * (1.0f - alpha);
      // next_T is never NaN (alpha = min(0.99, .) is not, and T only takes
      // values above the threshold), so one comparison decides both ways
      const bool live = next_T > kTransmittanceThreshold;
      done = done || (pass && !live);
      if (pass && live) {
        const float vis = alpha * T;
        if constexpr (CH > 0) {
          const float col[4] = {xc.z, xc.w, ex.x, ex.y};
#pragma unroll
          for (int c = 0; c < CH; ++c) acc[c] = __builtin_fmaf(col[c], vis, acc[c]);
        } else {
          const float* colp = a.colors + static_cast<int64_t>(__float_as_int(xc.z)) * channels;
          for (int c = 0; c < channels; ++c) acc[c] += colp[c] * vis;
        }
        cur = static_cast<int32_t>(b0 + k);
        T = next_T;
      }
    };
    auto falloff = [&](const float4& co, const float4& xc, bool* pass, float* alpha) {
      const float dx = xc.x - px;
      const float dy = xc.y - py;
      const float sigma = (co.x * dx * dx + co.z * dy * dy) + co.y * dx * dy;  // co.x, co.z pre-halved
      *alpha = fminf(kMaxAlpha, co.w * exp_alpha(-sigma));
      *pass = !(sigma < 0.0f || *alpha < kAlphaThreshold);
    };
    auto load = [&](int k, float4& co, float4& xc, float4& ex) {
      const float4* rec = reinterpret_cast<const float4*>(s_rec + k * FW);
      co = rec[0];
      xc = rec[1];
      if constexpr (FW > 8) ex = rec[2];
    };
    for (int c0 = 0; c0 < cnt; c0 += kWave) {
      // records of this 64-slot chunk that may touch this wave (all lanes vote)
      const int kl = c0 + lane;
      const uint32_t mk = kl < cnt ? s_mask[kl] : 0u;
      const bool mine = (mk >> wave) & 1u;
      uint64_t bits = __ballot(mine);
      if (__ballot(!done) == 0) bits = 0;  // every pixel of the wave has saturated
      while (bits) {
        const int k1 = c0 + __builtin_ctzll(bits);
        bits &= bits - 1;
        const bool two = bits != 0;
        const int k2 = two ? c0 + __builtin_ctzll(bits) : k1;
        bits &= bits - 1;
        float4 co1, xc1, ex1 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float4 co2, xc2, ex2 = ex1;
        load(k1, co1, xc1, ex1);
        load(k2, co2, xc2, ex2);
        bool p1, p2;
        float al1, al2;
        falloff(co1, xc1, &p1, &al1);
        falloff(co2, xc2, &p2, &al2);
        composite(k1, xc1, ex1, p1, al1);
        composite(k2, xc2, ex2, p2 && two, al2);
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

// Wave-wide sums of N values per lane by transposition (gfx950): three
// exchange levels halve the number of live values while doubling the lanes
// each one covers -- permlane32_swap (lane ^ 32), permlane16_swap (lane ^ 16),
// DPP row_ror:8 (lane ^ 8) -- then quad_perm / row_half_mirror DPP adds finish
// the sums inside each group of 8 lanes. A pair (a, b) at a level leaves the
// sum of a on lanes whose level bit is 0 and of b where it is 1; an unpaired
// last value is summed on its bit-0 side only at the permlane levels (its
// partner register holds a dead value) and on both sides at the DPP level. After the call, value y[m] on a lane with bits
// h = lane[5], r = lane[4], e = lane[3] is the wave total of input
// red_index<N>(m, h, r, e) (N: not a total, to be discarded); all 8 lanes of
// a group hold the same values.
// Costs about 2.3 VALU per value instead of 6 DPP steps per value.
template <int N>
struct Red {
  static constexpr int NA = (N + 1) / 2;   // after lane ^ 32
  static constexpr int NB = (NA + 1) / 2;  // after lane ^ 16
  static constexpr int NC = (NB + 1) / 2;  // after lane ^ 8
};

// Input index of y[m] on a lane with bits (h, r, e), or N where that lane's
// y[m] is not a total: an unpaired value at the permlane levels is exchanged
// with a dead register (no copy), so only its bit-0 side holds its sum.
template <int N>
__device__ __forceinline__ int red_index(int m, int h, int r, int e) {
  int c = 2 * m + e;
  if (c >= Red<N>::NB) c = 2 * m;
  const int b = 2 * c + r;
  if (b >= Red<N>::NA) return N;
  const int v = 2 * b + h;
  return v < N ? v : N;
}

__device__ __forceinline__ float fbits(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ unsigned ubits(float f) { return __builtin_bit_cast(unsigned, f); }

template <int N>
__device__ __forceinline__ void wave_transpose_reduce(const float (&v)[N], float (&y)[Red<N>::NC], bool e_bit) {
  constexpr int NA = Red<N>::NA, NB = Red<N>::NB, NC = Red<N>::NC;
  static_assert(N >= 3, "the unpaired exchange reuses the previous pair's register");
  // the unpaired value's partner is the previous pair's second swap output,
  // dead once added, so no register is copied for it
  float w[NA];
  unsigned spare = 0u;
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const unsigned b = (2 * i + 1 < N) ? ubits(v[2 * i + 1]) : spare;
    const auto sw = __builtin_amdgcn_permlane32_swap(ubits(v[2 * i]), b, false, false);
    w[i] = fbits(sw[0]) + fbits(sw[1]);
    spare = sw[1];
  }
  float x[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const unsigned b = (2 * i + 1 < NA) ? ubits(w[2 * i + 1]) : spare;
    const auto sw = __builtin_amdgcn_permlane16_swap(ubits(w[2 * i]), b, false, false);
    x[i] = fbits(sw[0]) + fbits(sw[1]);
    spare = sw[1];
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const float a = x[2 * i];
    if (2 * i + 1 < NB) {
      const float b = x[2 * i + 1];
      const float send = e_bit ? a : b;
      const float keep = e_bit ? b : a;
      y[i] = keep + fbits(__builtin_amdgcn_update_dpp(0u, ubits(send), 0x128, 0xf, 0xf, false));  // row_ror:8
    } else {
      y[i] = a + fbits(__builtin_amdgcn_update_dpp(0u, ubits(a), 0x128, 0xf, 0xf, false));
    }
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) y[i] += fbits(__builtin_amdgcn_update_dpp(0u, ubits(y[i]), 0xB1, 0xf, 0xf, false));   // lane ^ 1
#pragma unroll
  for (int i = 0; i < NC; ++i) y[i] += fbits(__builtin_amdgcn_update_dpp(0u, ubits(y[i]), 0x4E, 0xf, 0xf, false));   // lane ^ 2
#pragma unroll
  for (int i = 0; i < NC; ++i) y[i] += fbits(__builtin_amdgcn_mov_dpp(ubits(y[i]), 0x141, 0xf, 0xf, true));  // 7 - lane
}

// Backward. One block per tile, in the heavy-first tile order of `order`
// (see below); one lane owns one pixel of the tile (blocks are padded to
// whole wave64s; padding lanes own nothing). The tile's list is walked
// back-to-front in batches of BB entries from the tile's largest last_id; the
// next batch's records are loaded into registers while the current one is
// processed, and each staged record carries its per-wave touch mask. For each
// entry a wave visits (ballot over 64 slots, past-last and culled entries
// skipped), every lane computes its pixel's partial gradients in a reduced
// basis (below); a wave with a contributing lane sums them over the wave
// (wave_transpose_reduce) and one lane per 8-lane group stores its totals
// into the wave's accumulator slot for that entry (plain LDS stores; each
// (wave, entry) slot is written at most once per batch). After the batch the
// block adds up the per-wave slots, maps them back to gradients and flushes
// one global atomic per (entry, nonzero component).
//
// Per pixel, with the reference's per-channel `buffer` (gsplat_rasterize.cpp:
// 500-546) folded into B = sum_c buffer_c * v_rc_c and D = sum_c col_c * v_rc_c:
//   v_alpha = T D + ra (coef - B),  B += fac D,
// and the geometry gradients accumulated as h = v_sigma * (dx, dy):
//   v_conic = (hx dx / 2, hx dy, hy dy / 2),  v_mean2d = conic * (sum hx, sum hy)
// (the conic is the same for every pixel of an entry, so it is applied once
// after the reduction). Accumulated components: colors (CH), hx dx, hx dy,
// hy dy, hx, hy, vis * v_alpha, and |v_mean2d| per pixel (x, y) with absgrad.
// The contribution is computed on every lane of a visiting wave and selected
// to zero where the pixel does not contribute (no branches, no accumulators
// to clear). CH == 0 (runtime channel count) sends colour gradients straight
// to global memory.
// Six waves per SIMD (at most 80 VGPRs) where that needs no spills: one to
// three channels without absgrad (the training path); the register need
// leaves the others as they are.
constexpr int bwd_min_waves(int ch, bool abs) { return (!abs && ch >= 1 && ch <= 3) ? 6 : 1; }
// s_waitcnt immediate (gfx9 encoding): vmcnt 0 (bits 3:0 and 15:14), expcnt 7
// (bits 6:4) and lgkmcnt 15 (bits 11:8), i.e. wait for vector memory only
constexpr int kWaitVmemOnly = 0x0F70;
// flush lanes per entry (output components: CH colours, 3 conic, 2 mean, 1
// opacity, 2 |mean| with absgrad: at most 12) and the kinds of component
constexpr int kFlushLanes = 16;
constexpr int kFlushPlain = 0, kFlushMean = 1, kFlushOpacity = 2;

template <int CH, bool ABS>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(bwd_min_waves(CH, ABS))))
raster_bwd_kernel(
    RasterArgs a, int BB, int64_t n_units, const int32_t* __restrict__ order, const int32_t* __restrict__ cost,
    const float* __restrict__ render_alphas, const int32_t* __restrict__ last_ids,
    const float* __restrict__ v_render_colors, const float* __restrict__ v_render_alphas,
    float* __restrict__ v_means2d_abs, float* __restrict__ v_means2d, float* __restrict__ v_conics,
    float* __restrict__ v_colors, float* __restrict__ v_opacities, float* __restrict__ v_backgrounds) {
  constexpr int LC = CH > 0 ? CH : 1;
  constexpr int AC = CH > 0 ? CH : kMaxChannels;
  constexpr int NG = ABS ? 8 : 6;  // geometry components
  constexpr int NV = (CH > 0 ? CH : 0) + NG;
  constexpr int o = CH > 0 ? CH : 0;  // first geometry component
  constexpr int NC = Red<2 * NV>::NC;  // sums per lane of a record pair's reduction
  constexpr int NS = NV + 1;  // accumulator words per (wave, slot); the last takes discarded values
  constexpr int RW = bwd_record_words(CH);
  extern __shared__ float smem[];
  const int BS = blockDim.x;
  const int n_waves = BS / kWave;
  // one record per batch slot, read through a single address: conic xyz +
  // opacity, mean xy, colours (CH > 0), Gaussian id, per-wave touch bits
  constexpr int GW = 6 + o;  // word of the Gaussian id; the touch mask follows
  float* s_rec = smem;                  // [BB][RW]
  float* s_acc = smem + RW * BB;        // [n_waves][BB][NS]
  float4* s_rect = reinterpret_cast<float4*>(s_acc + n_waves * BB * NS);  // [n_waves] wave pixel rects
  auto s_g = [&](int k) { return __float_as_int(s_rec[k * RW + GW]); };
  auto s_mask = [&](int k) { return __float_as_uint(s_rec[k * RW + GW + 1]); };

  const int channels = CH > 0 ? CH : a.channels;
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const bool e_bit = (lane >> 3) & 1;
  const bool red_slot = (lane & 7) == 7;  // lane 7 of each 8-lane group stores
  const bool second_half = (lane >> 5) & 1;  // holds the pair's second record's sums
  // this lane's accumulator words for entry slot 0 (slot k adds k * NS): the
  // pair reduction's input 2 i + h is component i of record h, h = lane bit 5;
  // inputs that are not totals on this lane go to the discard word NV
  float* red_at[NC];
#pragma unroll
  for (int m = 0; m < NC; ++m) {
    const int in = red_index<2 * NV>(m, (lane >> 5) & 1, (lane >> 4) & 1, (lane >> 3) & 1);
    red_at[m] = s_acc + wave * BB * NS + (in < 2 * NV ? in / 2 : NV);
  }
  const int64_t n_tiles = static_cast<int64_t>(a.tw) * a.th;
  const int acc_words = n_waves * BB * NS;
  // this thread's flush role (the same for every slot it flushes, as the
  // block size is a multiple of kFlushLanes): output component c = t % 16 of
  // an entry, read from accumulator word(s) fl_word0 (fl_word1) and added to
  // fl_base[g * fl_stride + fl_comp]
  const int fc = t % kFlushLanes;
  int fl_word0 = -1, fl_word1 = -1, fl_kind = kFlushPlain, fl_comp = 0, fl_stride = 1;
  float fl_scale = 1.0f;
  float* fl_base = v_opacities;
  if (fc < (CH > 0 ? CH : 0)) {
    fl_word0 = fc, fl_base = v_colors, fl_stride = CH, fl_comp = fc;
  } else if (fc < o + 3) {
    fl_word0 = fc, fl_base = v_conics, fl_stride = 3, fl_comp = fc - o, fl_scale = fc - o == 1 ? 1.0f : 0.5f;
  } else if (fc < o + 5) {
    fl_word0 = o + 3, fl_word1 = o + 4, fl_kind = kFlushMean, fl_base = v_means2d, fl_stride = 2, fl_comp = fc - o - 3;
  } else if (fc == o + 5) {
    fl_word0 = o + 5, fl_kind = kFlushOpacity, fl_base = v_opacities;
  } else if (ABS && fc < o + 8) {
    fl_word0 = fc, fl_base = v_means2d_abs, fl_stride = 2, fl_comp = fc - o - 6;
  }

  // One block per tile, launched in the cost-sorted order: block b takes the
  // tile at rank b. The dispatcher starts blocks in index order as resident
  // blocks finish, so the heaviest tiles start first and the launch ends on
  // the lightest (longest-first balancing done by the hardware; a persistent
  // grid dealing about three tiles per block, statically or from a shared
  // counter, left CUs idle while their last blocks finished).
  {
    const int64_t unit = blockIdx.x;
    if (unit >= n_units) return;  // uniform across the block
    const int64_t it = order[unit];
    const int64_t image = it / n_tiles;
    const int tile = static_cast<int>(it % n_tiles);
    const int tx = tile % a.tw, ty = tile / a.tw;
    // masked tiles contribute nothing; their cost is 0, so the walk is empty
    int64_t start, end;
    tile_range(a, image, tile, &start, &end);
    // the tile's replay length (largest last_id - start + 1) from the schedule
    // pass; the first batch is fetched before the pixel state is read
    const int64_t stop = start + cost[it];
    // Register pipeline of batch records (lanes t < BB; slot t of the batch
    // [lo, hi) holds entry hi - 1 - t, back to front): the flatten ids are
    // loaded two batches ahead and the records one batch ahead, and nothing
    // waits for them until the batch is staged, where the touch mask is
    // formed. Ids outside [0, G) stage a zero-opacity record (never
    // contributes) and no colour read.
    int32_t r_id = 0;
    float2 r_xy = make_float2(0.0f, 0.0f);
    float4 r_co = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int32_t r_g = 0;
    float r_col[LC];
    auto load_ids = [&](int64_t hi, int64_t lo) {
      const int64_t j = hi - 1 - t;
      if (t < BB && j >= lo) r_id = a.flatten_ids[j];
    };
    auto load_records = [&](int64_t hi, int64_t lo) {  // of the ids in r_id
      const int64_t j = hi - 1 - t;
      if (t < BB && j >= lo) {
        const int32_t g = r_id;
        const bool ok = g >= 0 && static_cast<int64_t>(g) < a.G;
        const int64_t gg = ok ? g : 0;
        r_g = ok ? g : 0;
        if (ok) {
          r_xy = make_float2(a.means2d[gg * 2], a.means2d[gg * 2 + 1]);
          r_co = make_float4(a.conics[gg * 3], a.conics[gg * 3 + 1], a.conics[gg * 3 + 2], a.opacities[gg]);
        } else {
          r_xy = make_float2(0.0f, 0.0f);
          r_co = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if constexpr (CH > 0) {
#pragma unroll
          for (int c = 0; c < CH; ++c) r_col[c] = ok ? a.colors[gg * CH + c] : 0.0f;
        }
      }
    };
    if (stop > start) {
      const int64_t lo0 = max<int64_t>(start, stop - BB);
      load_ids(stop, lo0);
      load_records(stop, lo0);
      if (lo0 > start) load_ids(lo0, max<int64_t>(start, lo0 - BB));
    }

    store_wave_rects(s_rect, n_waves, a.ts, tx, ty);  // read after the batch loop's first barrier
    int qx, qy;
    lane_pixel(t, a.ts, &qx, &qy);
    const int x = tx * a.ts + qx;
    const int y = ty * a.ts + qy;
    const bool inside = t < a.ts * a.ts && x < a.W && y < a.H;
    const int64_t pix = (image * a.H + y) * static_cast<int64_t>(a.W) + x;
    const float px = static_cast<float>(x) + 0.5f;
    const float py = static_cast<float>(y) + 0.5f;
    const float T_final = inside ? 1.0f - render_alphas[pix] : 1.0f;
    float T = T_final;
    int last_rel = -1;  // last contributor relative to start, -1 for none
    if (inside) {
      const int64_t l = min<int64_t>(end - 1, last_ids[pix]) - start;
      last_rel = static_cast<int>(max<int64_t>(-1, min<int64_t>(l, INT32_MAX)));
    }
    float v_rc[AC];
    float bg_dot = 0.0f;
    for (int c = 0; c < channels; ++c) v_rc[c] = inside ? v_render_colors[pix * channels + c] : 0.0f;
    const float v_ra = inside && v_render_alphas ? v_render_alphas[pix] : 0.0f;
    if (a.backgrounds) {
      const float* bg = a.backgrounds + image * channels;
      for (int c = 0; c < channels; ++c) bg_dot += bg[c] * v_rc[c];
    }
    // d(final-transmittance terms)/d(alpha) = ra * coef
    const float coef = T_final * v_ra + -T_final * bg_dot;
    float Bc = coef;  // coef - B, B the running colour buffer (starts at 0)
    // the wave's colour cotangents and final transmittances are all finite
    // (then a lane that does not contribute can add fac * v_rc = 0 without a
    // select)
    bool rc_finite = fabsf(T_final) <= 3.402823466e38f;
    for (int c = 0; c < channels; ++c) rc_finite = rc_finite && fabsf(v_rc[c]) <= 3.402823466e38f;
    const bool wave_rc_finite = __ballot(!rc_finite) == 0;
    // entries past every pixel of the wave's last contributor are skipped
    int wave_last = last_rel;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) wave_last = max(wave_last, __shfl_xor(wave_last, off, kWave));


    for (int64_t b1 = stop; b1 > start; b1 -= BB) {
      const int64_t b0 = max<int64_t>(start, b1 - BB);
      __syncthreads();  // previous batch fully consumed and flushed
      if (t < BB && b1 - 1 - t >= b0) {
        const uint32_t r_mask = touch_mask(r_xy, r_co, n_waves, s_rect);
        float* rec = s_rec + t * RW;
        // conic diagonal pre-halved, as in the forward (the same sigma bit for
        // bit); the flush and the absolute gradients double it back exactly
        *reinterpret_cast<float4*>(rec) = make_float4(0.5f * r_co.x, r_co.y, 0.5f * r_co.z, r_co.w);
        float tail[RW - 4];
#pragma unroll
        for (int i = 0; i < RW - 4; ++i) tail[i] = 0.0f;
        tail[0] = r_xy.x;
        tail[1] = r_xy.y;
        if constexpr (CH > 0) {
#pragma unroll
          for (int c = 0; c < CH; ++c) tail[2 + c] = r_col[c];
        }
        tail[GW - 4] = __int_as_float(r_g);
        bool rec_finite = fabsf(r_xy.x) <= 3.402823466e38f && fabsf(r_xy.y) <= 3.402823466e38f;
        if constexpr (CH > 0) {
#pragma unroll
          for (int c = 0; c < CH; ++c) rec_finite = rec_finite && fabsf(r_col[c]) <= 3.402823466e38f;
        }
        tail[GW - 3] = __uint_as_float(r_mask | (rec_finite ? 0u : kNonFiniteRecord));
#pragma unroll
        for (int i = 0; i < RW - 4; i += 4)
          *reinterpret_cast<float4*>(rec + 4 + i) = make_float4(tail[i], tail[i + 1], tail[i + 2], tail[i + 3]);
      }
      // acc_words is a multiple of 4 (BB is a multiple of 64)
      for (int w = t * 4; w < acc_words; w += BS * 4)
        *reinterpret_cast<float4*>(s_acc + w) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      __syncthreads();
      // the next batch's records and the ids of the batch after it, in flight
      // during this one
      if (b0 > start) {
        const int64_t lo1 = max<int64_t>(start, b0 - BB);
        load_records(b0, lo1);
        if (lo1 > start) load_ids(lo1, max<int64_t>(start, lo1 - BB));
      }
      const int cnt = static_cast<int>(b1 - b0);
      const int k_rel0 = static_cast<int>(b1 - 1 - start);  // entry of slot 0, relative to start
      // Visits come in pairs of straight-line code so that the two records'
      // falloff, alpha and gradient terms overlap and their wave sums are
      // one reduction; only transmittance T and the buffer (Bc) pass from the
      // first visit to the second (list order, back to front). A chunk with
      // an odd number of visits ends with an inert second visit: no lane
      // valid, its sums not stored.
      struct Fall {
        float dx, dy, vis, a_raw, alpha;
        bool valid;
      };
      // falloff of this lane's pixel under the record of slot k (co: conic +
      // opacity, xc: mean xy + colours 0-1, ex: colours 2-3 when CH > 2)
      auto falloff = [&](int k, const float4& co, const float4& xc) {
        Fall f;
        const int k_rel = k_rel0 - k;
        f.dx = xc.x - px;
        f.dy = xc.y - py;
        const float sigma = (co.x * f.dx * f.dx + co.z * f.dy * f.dy) + co.y * f.dx * f.dy;  // co.x, co.z pre-halved
        f.vis = exp_alpha(-sigma);
        f.a_raw = co.w * f.vis;
        f.alpha = fminf(kMaxAlpha, f.a_raw);
        f.valid = k_rel <= last_rel && !(sigma < 0.0f || f.alpha < kAlphaThreshold);
        return f;
      };
      // this lane's partial gradients for slot k (v, reduced by the caller)
      auto contribute = [&](int k, const float4& co, const float4& xc, const float4& ex, const Fall& f,
                            bool store, bool careful, float (&v)[NV]) {
        const bool valid = f.valid;
        // A lane that does not contribute takes ra = 1 and alpha = 0, so T
        // stays exactly T and fac is 0; the geometry terms are still
        // selected, and (careful: the chunk holds a record with a non-finite
        // mean or colour, or the wave a non-finite colour cotangent) so are
        // the colour terms, the buffer update and the offsets, so non-finite
        // values of the record or of a pixel's cotangent never reach another
        // pixel's sums. Otherwise D is finite and fac D is exactly 0 for such
        // a lane, which leaves the buffer as it is without a select.
        const float ra = valid ? __builtin_amdgcn_rcpf(fmaxf(kMinOneMinusAlpha, 1.0f - f.alpha)) : 1.0f;
        const float T_new = T * ra;
        const float fac = (valid ? f.alpha : 0.0f) * T_new;
        float D;
        if constexpr (CH > 0) {
          D = xc.z * v_rc[0];
          v[0] = (careful && !valid) ? 0.0f : fac * v_rc[0];
#pragma unroll
          for (int c = 1; c < CH; ++c) {
            const float colc = c == 1 ? xc.w : (c == 2 ? ex.x : ex.y);
            D = __builtin_fmaf(colc, v_rc[c], D);
            v[c] = (careful && !valid) ? 0.0f : fac * v_rc[c];
          }
        } else {
          const int64_t gg = s_g(k);
          const float* gcol = a.colors + gg * channels;
          D = 0.0f;
          for (int c = 0; c < channels; ++c) D = __builtin_fmaf(gcol[c], v_rc[c], D);
          for (int c = 0; c < channels; ++c) {
            const float sum = wave_sum_uniform(valid ? fac * v_rc[c] : 0.0f);
            if (store && lane == 0 && sum != 0.0f) unsafeAtomicAdd(v_colors + gg * channels + c, sum);
          }
        }
        // Bc = coef - B, the reference's (coef - B) with B its running buffer
        const float v_alpha = __builtin_fmaf(T_new, D, ra * Bc);
        Bc = (CH == 0 || careful) ? (valid ? __builtin_fmaf(-fac, D, Bc) : Bc) : __builtin_fmaf(-fac, D, Bc);
        T = T_new;
        const bool geo = valid && f.a_raw <= kMaxAlpha;
        const float v_sigma = geo ? -f.a_raw * v_alpha : 0.0f;
        const float gx = (careful && !geo) ? 0.0f : f.dx;
        const float gy = (careful && !geo) ? 0.0f : f.dy;
        const float hx = v_sigma * gx;
        const float hy = v_sigma * gy;
        v[o + 0] = hx * gx;
        v[o + 1] = hx * gy;
        v[o + 2] = hy * gy;
        v[o + 3] = hx;
        v[o + 4] = hy;
        // vis v_alpha = -v_sigma / opacity: the flush divides the sum once
        v[o + 5] = v_sigma;
        if constexpr (ABS) {
          v[o + 6] = geo ? fabsf(__builtin_fmaf(co.x + co.x, hx, co.y * hy)) : 0.0f;
          v[o + 7] = geo ? fabsf(__builtin_fmaf(co.y, hx, (co.z + co.z) * hy)) : 0.0f;
        }
      };
      auto load = [&](int k, float4& co, float4& xc, float4& ex) {
        const float4* rec = reinterpret_cast<const float4*>(s_rec + k * RW);
        co = rec[0];
        xc = rec[1];
        if constexpr (RW > 8) ex = rec[2];
      };
      for (int c0 = 0; c0 < cnt; c0 += kWave) {
        // slots of this chunk that may touch this wave and are not past its
        // last contributor (all lanes vote)
        const int kl = c0 + lane;
        const uint32_t mk = kl < cnt ? s_mask(kl) : 0u;
        const bool mine = k_rel0 - kl <= wave_last && ((mk >> wave) & 1u);
        uint64_t bits = __ballot(mine);
        const bool careful = !wave_rc_finite || __ballot(mine && (mk & kNonFiniteRecord)) != 0;
        while (bits) {
          const int k1 = c0 + __builtin_ctzll(bits);
          bits &= bits - 1;
          const bool two = bits != 0;
          const int k2 = two ? c0 + __builtin_ctzll(bits) : k1;
          bits &= bits - 1;
          float4 co1, xc1, ex1 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          float4 co2, xc2, ex2 = ex1;
          load(k1, co1, xc1, ex1);
          load(k2, co2, xc2, ex2);
          const Fall f1 = falloff(k1, co1, xc1);
          Fall f2 = falloff(k2, co2, xc2);
          f2.valid = f2.valid && two;
          float v1[NV], v2[NV];
          if (careful) {
            contribute(k1, co1, xc1, ex1, f1, true, true, v1);
            contribute(k2, co2, xc2, ex2, f2, two, true, v2);
          } else {
            contribute(k1, co1, xc1, ex1, f1, true, false, v1);
            contribute(k2, co2, xc2, ex2, f2, two, false, v2);
          }
          // interleaved, so lanes 0-31 end with the first record's sums and
          // lanes 32-63 with the second's
          float vv[2 * NV], y[NC];
#pragma unroll
          for (int i = 0; i < NV; ++i) {
            vv[2 * i] = v1[i];
            vv[2 * i + 1] = v2[i];
          }
          wave_transpose_reduce<2 * NV>(vv, y, e_bit);
          if (red_slot && (two || !second_half)) {
            // 24-bit multiply: full rate, unlike a 32-bit one (slots < BB)
            const int off = __mul24(second_half ? k2 : k1, NS);
#pragma unroll
            for (int mm = 0; mm < NC; ++mm) red_at[mm][off] = y[mm];
          }
        }
      }
      __syncthreads();
      // The vector memory counter counts loads, stores and atomics in issue
      // order, so the loaders' wait for the next batch's records (issued
      // before the visits) would also wait for the atomics below. Waiting for
      // vector memory here, before the atomics, leaves those records ready.
      __builtin_amdgcn_s_waitcnt(kWaitVmemOnly);
      // Flush: 16 lanes per slot, lane c of the group adds output component
      // c of the slot's entry (summed over the waves), so one atomic
      // instruction covers four entries and each entry's colours, conic and
      // mean are each one cache line: the memory system serves atomics per
      // cache line, whatever the number of lanes that hit it.
      for (int idx = t; idx < cnt * kFlushLanes; idx += BS) {
        const int slot = idx / kFlushLanes;
        if (fl_word0 < 0) continue;  // lanes past the slot's components
        float v = 0.0f, v2 = 0.0f;
        for (int w = 0; w < n_waves; ++w) {
          v += s_acc[(w * BB + slot) * NS + fl_word0];
          if (fl_word1 >= 0) v2 += s_acc[(w * BB + slot) * NS + fl_word1];
        }
        const int64_t gg = s_g(slot);
        if (fl_kind == kFlushMean) {
          // v_mean2d = conic (sum hx, sum hy); the conic applies only to
          // geometry terms some pixel produced: with none, the reference adds
          // nothing, even for a non-finite conic (0 * NaN would otherwise
          // reach the mean's gradient)
          if (v == 0.0f && v2 == 0.0f) continue;
          const float4 co = *reinterpret_cast<const float4*>(s_rec + slot * RW);
          v = fl_comp == 0 ? (co.x + co.x) * v + co.y * v2 : co.y * v + (co.z + co.z) * v2;
        } else if (fl_kind == kFlushOpacity) {
          // sum of v_sigma = -opacity vis v_alpha: the opacity is at least
          // 1/255 wherever a pixel contributed (alpha passed the threshold)
          if (v == 0.0f) continue;
          v = -v / s_rec[slot * RW + 3];
        } else {
          v *= fl_scale;
        }
        if (v != 0.0f) unsafeAtomicAdd(fl_base + gg * fl_stride + fl_comp, v);
      }
    }
  }
}

// Heavy-first tile schedule for the backward. A tile's cost is the number of
// list entries its pixels replay (largest last_id - start + 1, 0 when masked
// or empty). The backward launches one block per tile in descending cost
// order, so the longest tiles start first and the end of the launch is made
// of short ones (greedy longest-processing-time scheduling).
//
// The same pass over the tile's pixels also forms the tile's share of the
// background gradient, v_backgrounds[i, c] = sum over the unmasked pixels of
// image i of (1 - render_alpha) * v_render_colors[c] (gsplat_rasterize.cpp:
// 459-464; the background enters each pixel as T_final * bg): one partial
// per (tile, channel), summed per image by the order kernel's extra blocks.
// No atomics: every partial has one writer.
constexpr int kCostBuckets = 4096;  // costs >= 4095 share the heaviest bucket

template <int CH>
__global__ void __launch_bounds__(256) tile_cost_kernel(RasterArgs a, const int32_t* __restrict__ last_ids,
                                                        const float* __restrict__ render_alphas,
                                                        const float* __restrict__ v_render_colors,
                                                        int32_t* __restrict__ cost, float* __restrict__ bg_part,
                                                        ZeroSpans zero) {
  constexpr int LC = CH > 0 ? CH : 1;
  __shared__ int s_best[256 / kWave];
  __shared__ float s_sum[256 / kWave][LC];
  const int tx = blockIdx.x, ty = blockIdx.y;
  const int64_t image = blockIdx.z;
  const int tile = ty * a.tw + tx;
  const int64_t n_tiles = static_cast<int64_t>(a.tw) * a.th;
  const int64_t unit = image * n_tiles + tile;
  const int t = threadIdx.x;
  const int channels = CH > 0 ? CH : a.channels;
  // the backward's accumulated outputs start at zero: cleared here, one
  // launch ahead of the kernel that accumulates into them
  zero_spans_share(zero, unit * 256 + t, static_cast<int64_t>(a.I) * n_tiles * 256);
  int64_t start, end;
  tile_range(a, image, tile, &start, &end);
  const bool live = !(a.masks && !a.masks[unit]);
  int best = 0;
  float acc[LC];
#pragma unroll
  for (int c = 0; c < LC; ++c) acc[c] = 0.0f;
  if (live) {
    for (int q = t; q < a.ts * a.ts; q += 256) {
      const int x = tx * a.ts + q % a.ts;
      const int y = ty * a.ts + q / a.ts;
      if (x >= a.W || y >= a.H) continue;
      const int64_t pix = (image * a.H + y) * static_cast<int64_t>(a.W) + x;
      const int64_t last = min<int64_t>(end - 1, last_ids[pix]);
      best = max(best, static_cast<int>(min<int64_t>(max<int64_t>(last - start + 1, 0), INT32_MAX)));
      if constexpr (CH > 0) {
        if (bg_part) {
          const float T_final = 1.0f - render_alphas[pix];
#pragma unroll
          for (int c = 0; c < CH; ++c) acc[c] += T_final * v_render_colors[pix * CH + c];
        }
      }
    }
  }
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) best = max(best, __shfl_xor(best, off, kWave));
  if (t % kWave == 0) s_best[t / kWave] = best;
  if (bg_part && CH > 0) {
#pragma unroll
    for (int c = 0; c < LC; ++c) {
      const float w = wave_sum_uniform(acc[c]);
      if (t % kWave == 0) s_sum[t / kWave][c] = w;
    }
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < 256 / kWave; ++w) best = max(best, s_best[w]);
    cost[unit] = best;
  }
  if (!bg_part) return;
  if constexpr (CH > 0) {
    if (t < CH) {
      float sum = 0.0f;
      for (int w = 0; w < 256 / kWave; ++w) sum += s_sum[w][t];
      bg_part[unit * CH + t] = sum;
    }
  } else {
    // any channel count: one channel at a time
    for (int c = 0; c < channels; ++c) {
      float v = 0.0f;
      if (live) {
        for (int q = t; q < a.ts * a.ts; q += 256) {
          const int x = tx * a.ts + q % a.ts;
          const int y = ty * a.ts + q / a.ts;
          if (x >= a.W || y >= a.H) continue;
          const int64_t pix = (image * a.H + y) * static_cast<int64_t>(a.W) + x;
          v += (1.0f - render_alphas[pix]) * v_render_colors[pix * channels + c];
        }
      }
      const float w = wave_sum_uniform(v);
      __syncthreads();  // the previous channel's partials have been read
      if (t % kWave == 0) s_sum[t / kWave][0] = w;
      __syncthreads();
      if (t == 0) {
        float sum = 0.0f;
        for (int k = 0; k < 256 / kWave; ++k) sum += s_sum[k][0];
        bg_part[unit * channels + c] = sum;
      }
    }
  }
}

// The same for 16-pixel tiles with a block per strip of kStripTiles tiles of
// one tile row: lane c of each wave takes pixel column c of the strip (so a
// wave reads 64 consecutive pixels of a row, 256-768 bytes, instead of four
// 16-pixel pieces), waves take rows w, w + 4, ...; each tile's values are
// reduced over its 16 lanes by DPP row shifts (one 16-lane row is one tile),
// then over the waves in LDS in a fixed order.
constexpr int kStripTiles = 4;

__device__ __forceinline__ float row16_sum(float v) {  // lane 15 of each 16-lane row: the row's sum
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x112, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x118, 0xf, 0xf, false));
  return v;
}

__device__ __forceinline__ int row16_max(int v) {  // lane 15 of each 16-lane row: the row's maximum (v >= 0)
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));
  return v;
}

template <int CH>
__global__ void __launch_bounds__(256) tile_cost_strip_kernel(RasterArgs a, const int32_t* __restrict__ last_ids,
                                                              const float* __restrict__ render_alphas,
                                                              const float* __restrict__ v_render_colors,
                                                              int32_t* __restrict__ cost, float* __restrict__ bg_part,
                                                              ZeroSpans zero) {
  static_assert(CH >= 1 && CH <= 4, "staged channel counts");
  constexpr int TS = 16, NW = 4;
  __shared__ int s_best[NW][kStripTiles];
  __shared__ float s_sum[NW][kStripTiles][CH];
  const int t = threadIdx.x, col = t % kWave, wave = t / kWave;
  const int64_t image = blockIdx.z;
  const int ty = blockIdx.y;
  const int k = col / TS;                        // tile of the strip
  const int tx = blockIdx.x * kStripTiles + k;   // its column in the tile grid
  const int64_t n_tiles = static_cast<int64_t>(a.tw) * a.th;
  const int64_t block = (image * gridDim.y + ty) * gridDim.x + blockIdx.x;
  zero_spans_share(zero, block * 256 + t, static_cast<int64_t>(gridDim.x) * gridDim.y * gridDim.z * 256);
  const bool tile_ok = tx < a.tw;
  const int64_t unit = image * n_tiles + static_cast<int64_t>(ty) * a.tw + tx;
  int64_t start = 0, end = 0;
  if (tile_ok) tile_range(a, image, ty * a.tw + tx, &start, &end);
  const bool live = tile_ok && !(a.masks && !a.masks[unit]);
  const int x = tx * TS + col % TS;
  int best = 0;
  float acc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) acc[c] = 0.0f;
  if (live && x < a.W) {
#pragma unroll
    for (int r = 0; r < TS / NW; ++r) {
      const int y = ty * TS + wave + NW * r;
      if (y >= a.H) break;
      const int64_t pix = (image * a.H + y) * static_cast<int64_t>(a.W) + x;
      const int64_t last = min<int64_t>(end - 1, last_ids[pix]);
      best = max(best, static_cast<int>(min<int64_t>(max<int64_t>(last - start + 1, 0), INT32_MAX)));
      if (bg_part) {
        const float T_final = 1.0f - render_alphas[pix];
#pragma unroll
        for (int c = 0; c < CH; ++c) acc[c] += T_final * v_render_colors[pix * CH + c];
      }
    }
  }
  best = row16_max(best);
#pragma unroll
  for (int c = 0; c < CH; ++c) acc[c] = row16_sum(acc[c]);
  if (col % TS == TS - 1) {
    s_best[wave][k] = best;
#pragma unroll
    for (int c = 0; c < CH; ++c) s_sum[wave][k][c] = acc[c];
  }
  __syncthreads();
  if (t < kStripTiles) {
    const int txo = blockIdx.x * kStripTiles + t;
    if (txo < a.tw) {
      const int64_t u = image * n_tiles + static_cast<int64_t>(ty) * a.tw + txo;
      int b = 0;
      float sum[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) sum[c] = 0.0f;
      for (int w = 0; w < NW; ++w) {
        b = max(b, s_best[w][t]);
#pragma unroll
        for (int c = 0; c < CH; ++c) sum[c] += s_sum[w][t][c];
      }
      cost[u] = b;
      if (bg_part) {
#pragma unroll
        for (int c = 0; c < CH; ++c) bg_part[u * CH + c] = sum[c];
      }
    }
  }
}

// Block 0: counting sort of the n tile costs into descending order. Blocks
// 1 .. I * channels (when bg_part is set): v_backgrounds[i][c] as the sum of
// image i's per-tile partials of channel c, in tile order (deterministic).
// Up to kOrderItems costs per thread are loaded at once and kept in registers
// for the second pass (n <= 8192 tiles); larger n loop over global memory.
constexpr int kOrderBlock = 1024;
constexpr int kOrderItems = 8;

__global__ void __launch_bounds__(kOrderBlock) tile_order_kernel(const int32_t* __restrict__ cost, int64_t n,
                                                                 int32_t* __restrict__ order,
                                                                 const float* __restrict__ bg_part, int64_t n_tiles,
                                                                 int channels, float* __restrict__ v_backgrounds) {
  static_assert(kCostBuckets % kOrderBlock == 0, "buckets per thread");
  constexpr int PER = kCostBuckets / kOrderBlock;
  constexpr int W = kOrderBlock / kWave;
  __shared__ int hist[kCostBuckets];
  __shared__ int s_w[W];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  if (blockIdx.x > 0) {
    const int64_t ic = blockIdx.x - 1;  // image * channels + c
    const int64_t image = ic / channels;
    const int c = static_cast<int>(ic % channels);
    const float* part = bg_part + image * n_tiles * channels + c;
    float v = 0.0f;
    for (int64_t j = t; j < n_tiles; j += kOrderBlock) v += part[j * channels];
    float* s_sum = reinterpret_cast<float*>(hist);
    const float w = wave_sum_uniform(v);
    if (lane == 0) s_sum[wave] = w;
    __syncthreads();
    if (t == 0) {
      float sum = 0.0f;
      for (int k = 0; k < W; ++k) sum += s_sum[k];
      v_backgrounds[ic] = sum;
    }
    return;
  }
  auto bucket = [](int32_t c) { return kCostBuckets - 1 - min(c, kCostBuckets - 1); };
  const bool in_regs = n <= static_cast<int64_t>(kOrderBlock) * kOrderItems;  // uniform
  int32_t b[kOrderItems];
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kOrderItems; ++k) {
      const int64_t i = t + static_cast<int64_t>(k) * kOrderBlock;
      b[k] = i < n ? bucket(cost[i]) : -1;
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) hist[t * PER + j] = 0;
  __syncthreads();
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kOrderItems; ++k)
      if (b[k] >= 0) atomicAdd(&hist[b[k]], 1);
  } else {
    for (int64_t i = t; i < n; i += kOrderBlock) atomicAdd(&hist[bucket(cost[i])], 1);
  }
  __syncthreads();
  int h[PER], sum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    h[j] = hist[t * PER + j];
    sum += h[j];
  }
  const int inc = wave_inclusive_scan(sum);
  if (lane == kWave - 1) s_w[wave] = inc;
  __syncthreads();
  int running = inc - sum;
#pragma unroll
  for (int w = 0; w < W; ++w) running += w < wave ? s_w[w] : 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    hist[t * PER + j] = running;
    running += h[j];
  }
  __syncthreads();
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kOrderItems; ++k)
      if (b[k] >= 0) order[atomicAdd(&hist[b[k]], 1)] = t + k * kOrderBlock;
  } else {
    for (int64_t i = t; i < n; i += kOrderBlock) order[atomicAdd(&hist[bucket(cost[i])], 1)] = static_cast<int32_t>(i);
  }
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }
// cost [n] int32, order [n] int32, background partials [n][channels] float
size_t bwd_workspace_bytes(int64_t n_tiles_total, int channels) {
  return 2 * align256(static_cast<size_t>(n_tiles_total) * 4) +
         align256(static_cast<size_t>(n_tiles_total) * channels * 4);
}

// records: mean 2, conic+opacity 4, colours (CH > 0), Gaussian id, touch mask
// plus one float4 wave rectangle per wave
size_t fwd_smem(int ch, int bs) {
  return static_cast<size_t>(bs) * (fwd_record_words(ch) + 1) * 4 + static_cast<size_t>(bs / kWave) * 16;
}
// Backward block: one pixel per lane, the whole tile in one block (measured
// fastest on gfx950 for 16x16 tiles against 2 or 4 pixels per lane and
// against splitting a tile over several blocks: the lower register count
// keeps six waves per SIMD resident). Batch length: 128 entries for blocks of
// up to 256 lanes, 64 above (bounds the per-wave accumulators to 52 KiB at
// 1024 lanes, 4 channels, absgrad); never more than the block, so one lane
// loads one record.
int bwd_block(int ts) { return (ts * ts + kWave - 1) / kWave * kWave; }
int bwd_batch(int bs) { return bs <= 128 ? bs : (bs <= 256 ? 128 : 64); }
// one record (bwd_record_words) per batch slot plus NV + 1 accumulator words
// per (wave, slot)
size_t bwd_smem(int ch, int bs, int bb, bool absgrad) {
  const int cc = ch > 0 ? ch : 0;
  const int ns = cc + (absgrad ? 8 : 6) + 1;
  return static_cast<size_t>(bb) * (bwd_record_words(ch) + (bs / kWave) * ns) * 4 + static_cast<size_t>(bs / kWave) * 16;
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

// ---------------------------------------------------------------------------
// Rasterize to indices (upstream gsplat's rasterize_to_indices_in_range,
// note/gsplat_cuda_source_map.md:494-545; the reference's planned
// rasterize_to_indices_3dgs_forward). Per pixel, starting from transmittance
// T0 (1 without a transmittance image), the entries of its tile's list at
// positions [range_start, range_end) that pass the forward's alpha test, in
// list order, until the next transmittance would fall to 1e-4 -- the
// forward's compositing rule with its alpha, threshold and exp, so the
// entries are exactly those the forward composites. One block per tile, one
// lane per pixel, records staged through LDS; pass 1 (WRITE false) counts
// per pixel, pass 2 writes each pixel's entries at its scanned start:
// gaussian id and the pixel's global index image * H * W + y * W + x.
template <bool WRITE>
__global__ void __launch_bounds__(1024) raster_indices_kernel(RasterArgs a, int64_t range_start, int64_t range_end,
                                                              const float* __restrict__ transmittances,
                                                              int32_t* __restrict__ counts,
                                                              const int32_t* __restrict__ starts, int64_t n_out,
                                                              int32_t* __restrict__ out_gauss,
                                                              int64_t* __restrict__ out_index) {
  __shared__ float4 s_co[1024];
  __shared__ float2 s_xy[1024];
  __shared__ int32_t s_g[1024];
  const int tx = blockIdx.x, ty = blockIdx.y;
  const int64_t image = blockIdx.z;
  const int t = threadIdx.x;
  const int bs = blockDim.x;
  const int x = tx * a.ts + t % a.ts, y = ty * a.ts + t / a.ts;
  const bool inside = t < a.ts * a.ts && x < a.W && y < a.H;
  const int64_t pix = image * a.H * a.W + static_cast<int64_t>(y) * a.W + x;
  int64_t s0, e0;
  tile_range(a, image, ty * a.tw + tx, &s0, &e0);
  const int64_t start = min(s0 + max<int64_t>(range_start, 0), e0);
  const int64_t end = min(s0 + max<int64_t>(range_end, 0), e0);
  const float px = static_cast<float>(x) + 0.5f, py = static_cast<float>(y) + 0.5f;
  float T = inside && transmittances ? transmittances[pix] : 1.0f;
  bool done = !inside;
  int32_t cnt = 0;
  int64_t pos = WRITE && inside ? starts[pix] : 0;
  for (int64_t b = start; b < end; b += bs) {
    if (__syncthreads_count(!done) == 0) break;
    const int64_t j = b + t;
    if (j < end) {
      float2 xy;
      float4 co;
      s_g[t] = load_gaussian(a, j, &xy, &co);
      s_xy[t] = xy;
      s_co[t] = co;
    }
    __syncthreads();
    const int n = static_cast<int>(min<int64_t>(bs, end - b));
    for (int k = 0; k < n && !done; ++k) {
      const float4 co = s_co[k];
      const float dx = s_xy[k].x - px;
      const float dy = s_xy[k].y - py;
      const float sigma = 0.5f * (co.x * dx * dx + co.z * dy * dy) + co.y * dx * dy;
      const float alpha = fminf(kMaxAlpha, co.w * exp_alpha(-sigma));
      if (sigma < 0.0f || alpha < kAlphaThreshold) continue;
      const float next_T = T * (1.0f - alpha);
      if (next_T <= kTransmittanceThreshold) {
        done = true;
        break;
      }
      if constexpr (WRITE) {
        if (pos < n_out) {
          out_gauss[pos] = s_g[k];
          out_index[pos] = pix;
        }
        ++pos;
      }
      ++cnt;
      T = next_T;
    }
  }
  if (!WRITE && inside) counts[pix] = cnt;
}

// E_f of the forward, per tile: the (pixel, list entry) evaluations of the
// reference's per-pixel loop (gsplat_rasterize.cpp:291-368) -- every entry of
// the pixel's tile list up to and including the one whose alpha would take
// the transmittance to 1e-4 -- summed over the tile's pixels into
// tile_evals[image, tile] (0 for a masked tile). The falloff, exp and
// thresholds are the forward's. This measures the work the rasterizer's
// roofline is priced on; the forward itself skips records that cannot touch a
// wave's pixels and stops at the block's last saturated pixel.
__global__ void __launch_bounds__(1024) raster_count_kernel(RasterArgs a, int64_t* __restrict__ tile_evals) {
  __shared__ float4 s_co[1024];
  __shared__ float2 s_xy[1024];
  __shared__ int64_t s_sum[1024 / kWave];
  const int tx = blockIdx.x, ty = blockIdx.y;
  const int64_t image = blockIdx.z;
  const int t = threadIdx.x;
  const int bs = blockDim.x;
  const int tile = ty * a.tw + tx;
  const int64_t n_tiles = static_cast<int64_t>(a.tw) * a.th;
  const int x = tx * a.ts + t % a.ts, y = ty * a.ts + t / a.ts;
  const bool inside = t < a.ts * a.ts && x < a.W && y < a.H;
  const bool masked = a.masks && !a.masks[image * n_tiles + tile];
  int64_t start, end;
  tile_range(a, image, tile, &start, &end);
  const float px = static_cast<float>(x) + 0.5f, py = static_cast<float>(y) + 0.5f;
  float T = 1.0f;
  bool done = !inside || masked;
  int64_t cnt = 0;
  for (int64_t b = start; b < end; b += bs) {
    if (__syncthreads_count(!done) == 0) break;
    const int64_t j = b + t;
    if (j < end) {
      float2 xy;
      float4 co;
      load_gaussian(a, j, &xy, &co);
      s_xy[t] = xy;
      s_co[t] = co;
    }
    __syncthreads();
    const int n = static_cast<int>(min<int64_t>(bs, end - b));
    for (int k = 0; k < n && !done; ++k) {
      ++cnt;
      const float4 co = s_co[k];
      const float dx = s_xy[k].x - px;
      const float dy = s_xy[k].y - py;
      const float sigma = 0.5f * (co.x * dx * dx + co.z * dy * dy) + co.y * dx * dy;
      const float alpha = fminf(kMaxAlpha, co.w * exp_alpha(-sigma));
      if (sigma < 0.0f || alpha < kAlphaThreshold) continue;
      const float next_T = T * (1.0f - alpha);
      if (next_T <= kTransmittanceThreshold) done = true;
      T = next_T;
    }
  }
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) cnt += __shfl_xor(cnt, off, kWave);
  if (t % kWave == 0) s_sum[t / kWave] = cnt;
  __syncthreads();
  if (t == 0) {
    int64_t sum = 0;
    for (int w = 0; w < bs / kWave; ++w) sum += s_sum[w];
    tile_evals[image * n_tiles + tile] = sum;
  }
}

// out[i] = exp_alpha(y[i]) (the rasterizer's exp, for unit tests).
__global__ void __launch_bounds__(256) exp_alpha_kernel(const float* __restrict__ y, int64_t n,
                                                        float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = exp_alpha(y[i]);
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" int gsplat_hip_rasterize_count_evals(const float* means2d, const float* conics, const float* opacities,
                                                const uint8_t* masks, const int32_t* tile_offsets,
                                                const int32_t* flatten_ids, int64_t I, int64_t G,
                                                int32_t image_width, int32_t image_height, int32_t tile_size,
                                                int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                                int64_t* tile_evals, void* stream) {
  RasterArgs a{means2d, conics, nullptr, opacities, nullptr, masks, tile_offsets, flatten_ids, G, 1,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects, G};
  int rc = check_args(a, "rasterize_count_evals");
  if (rc) return rc;
  if (G < 0) return invalid("rasterize_count_evals: invalid sizes.");
  if (I == 0 || tile_width == 0 || tile_height == 0) return GSPLAT_OK;
  if (!tile_offsets || !tile_evals || (n_isects > 0 && (!flatten_ids || !means2d || !conics || !opacities)))
    return invalid("rasterize_count_evals: null pointer.");
  const dim3 grid(tile_width, tile_height, static_cast<unsigned>(I));
  const int bs = (tile_size * tile_size + kWave - 1) / kWave * kWave;
  raster_count_kernel<<<grid, bs, 0, as_stream(stream)>>>(a, tile_evals);
  return check_launch("rasterize_count_evals");
}

extern "C" int gsplat_hip_exp_alpha_eval(const float* y, int64_t n, float* out, void* stream) {
  if (n < 0) return invalid("exp_alpha_eval: negative size.");
  if (n == 0) return GSPLAT_OK;
  if (!y || !out) return invalid("exp_alpha_eval: null pointer.");
  exp_alpha_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(y, n, out);
  return check_launch("exp_alpha_eval");
}

static int rasterize_fwd_impl(const float* means2d, const float* conics, const float* colors,
                              const float* opacities, const float* backgrounds, const uint8_t* masks,
                              const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I, int64_t N,
                              int64_t G, int32_t channels, int32_t image_width, int32_t image_height,
                              int32_t tile_size, int32_t tile_width, int32_t tile_height, int64_t n_isects,
                              float* render_colors, float* render_alphas, int32_t* last_ids, void* stream) {
  RasterArgs a{means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, N, channels,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects, G};
  if (G < 0) return invalid("rasterize_to_pixels_3dgs_forward: invalid sizes.");
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

static int rasterize_bwd_impl(const float* means2d, const float* conics, const float* colors,
                              const float* opacities, const float* backgrounds, const uint8_t* masks,
                              const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I, int64_t N,
                              int64_t G, int32_t channels, int32_t image_width, int32_t image_height,
                              int32_t tile_size, int32_t tile_width, int32_t tile_height, int64_t n_isects,
                              const float* render_alphas, const int32_t* last_ids, const float* v_render_colors,
                              const float* v_render_alphas, float* v_means2d_abs, float* v_means2d,
                              float* v_conics, float* v_colors, float* v_opacities, float* v_backgrounds,
                              void* workspace, size_t workspace_bytes, void* stream) {
  RasterArgs a{means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, N, channels,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects, G};
  int rc = check_args(a, "rasterize_to_pixels_3dgs_backward");
  if (rc) return rc;
  if (G < 0) return invalid("rasterize_to_pixels_3dgs_backward: invalid sizes.");
  if (!v_means2d || !v_conics || !v_colors || !v_opacities)
    return invalid("rasterize_to_pixels_3dgs_backward: null pointer.");
  if (backgrounds && !v_backgrounds) return invalid("rasterize_to_pixels_3dgs_backward: null v_backgrounds.");
  hipStream_t s = as_stream(stream);
  // outputs are accumulated from zero; the schedule kernel clears them
  // (v_backgrounds is written whole by the order kernel)
  const ZeroSpan spans[] = {{v_means2d, G * 2},
                            {v_conics, G * 3},
                            {v_colors, G * channels},
                            {v_opacities, G},
                            {v_means2d_abs, v_means2d_abs ? G * 2 : 0},
                            {v_backgrounds, backgrounds ? I * channels : 0}};
  if (I == 0 || tile_width == 0 || tile_height == 0) return fill_zero_spans(spans, 6, s);
  const ZeroSpans zero = pack_zero_spans(spans, 5);
  const dim3 grid(tile_width, tile_height, static_cast<unsigned>(I));
  if (!tile_offsets || !render_alphas || !last_ids || !v_render_colors ||
      (n_isects > 0 && (!flatten_ids || !means2d || !conics || !colors || !opacities)))
    return invalid("rasterize_to_pixels_3dgs_backward: null pointer.");
  const int ch = channels <= 4 ? channels : 0;
  const int bs = bwd_block(tile_size);
  const int64_t n_total = I * tile_width * static_cast<int64_t>(tile_height);
  if (n_total > INT32_MAX) return invalid("rasterize_to_pixels_3dgs_backward: too many tiles.");
  if (!workspace || workspace_bytes < bwd_workspace_bytes(n_total, channels)) {
    set_error("rasterize_to_pixels_3dgs_backward: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  int32_t* cost = static_cast<int32_t*>(workspace);
  int32_t* order = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + align256(n_total * 4));
  float* bg_part =
      backgrounds ? reinterpret_cast<float*>(static_cast<char*>(workspace) + 2 * align256(n_total * 4)) : nullptr;
  {
    KernelTimer timer("raster_bwd_schedule", s);
    const dim3 sgrid((tile_width + kStripTiles - 1) / kStripTiles, tile_height, static_cast<unsigned>(I));
    if (tile_size == 16 && ch >= 1) {  // strips of 16-pixel tiles
      switch (ch) {
        case 1: tile_cost_strip_kernel<1><<<sgrid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
        case 2: tile_cost_strip_kernel<2><<<sgrid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
        case 3: tile_cost_strip_kernel<3><<<sgrid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
        default: tile_cost_strip_kernel<4><<<sgrid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
      }
    } else {
      switch (ch) {
        case 1: tile_cost_kernel<1><<<grid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
        case 2: tile_cost_kernel<2><<<grid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
        case 3: tile_cost_kernel<3><<<grid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
        case 4: tile_cost_kernel<4><<<grid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
        default: tile_cost_kernel<0><<<grid, 256, 0, s>>>(a, last_ids, render_alphas, v_render_colors, cost, bg_part, zero); break;
      }
    }
    // block 0 orders the tiles; one more block per (image, channel) sums the background partials
    const unsigned order_blocks = 1 + (backgrounds ? static_cast<unsigned>(I * channels) : 0u);
    tile_order_kernel<<<order_blocks, kOrderBlock, 0, s>>>(cost, n_total, order, bg_part,
                                                          tile_width * static_cast<int64_t>(tile_height), channels,
                                                          v_backgrounds);
  }
  if ((rc = check_launch("rasterize_to_pixels_3dgs_backward"))) return rc;
  const int bb = bwd_batch(bs);
  const size_t sm = bwd_smem(ch, bs, bb, v_means2d_abs != nullptr);
  KernelTimer timer("raster_bwd", s);
  // one block per tile (block b: the tile of rank b in the heavy-first order)
#define GSPLAT_BWD_LAUNCH(C, ABS_, VABS)                                                                       \
  {                                                                                                            \
    const unsigned nb = static_cast<unsigned>(n_total);                                                        \
    raster_bwd_kernel<C, ABS_><<<nb, bs, sm, s>>>(a, bb, n_total, order, cost, render_alphas, last_ids,       \
                                                  v_render_colors, v_render_alphas, VABS, v_means2d, v_conics, \
                                                  v_colors, v_opacities, v_backgrounds);                        \
  }
#define GSPLAT_BWD_ABS(C)                            \
  if (v_means2d_abs) {                               \
    GSPLAT_BWD_LAUNCH(C, true, v_means2d_abs)        \
  } else {                                           \
    GSPLAT_BWD_LAUNCH(C, false, nullptr)             \
  }
  switch (ch) {
    case 1: GSPLAT_BWD_ABS(1); break;
    case 2: GSPLAT_BWD_ABS(2); break;
    case 3: GSPLAT_BWD_ABS(3); break;
    case 4: GSPLAT_BWD_ABS(4); break;
    default: GSPLAT_BWD_ABS(0); break;
  }
#undef GSPLAT_BWD_ABS
#undef GSPLAT_BWD_LAUNCH
  return check_launch("rasterize_to_pixels_3dgs_backward");
}

extern "C" int gsplat_hip_rasterize_fwd(const float* means2d, const float* conics, const float* colors,
                                        const float* opacities, const float* backgrounds, const uint8_t* masks,
                                        const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I, int64_t N,
                                        int32_t channels, int32_t image_width, int32_t image_height, int32_t tile_size,
                                        int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                        float* render_colors, float* render_alphas, int32_t* last_ids, void* stream) {
  return rasterize_fwd_impl(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, I, N,
                            I * N, channels, image_width, image_height, tile_size, tile_width, tile_height, n_isects,
                            render_colors, render_alphas, last_ids, stream);
}

extern "C" int gsplat_hip_rasterize_fwd_packed(const float* means2d, const float* conics, const float* colors,
                                               const float* opacities, const float* backgrounds,
                                               const uint8_t* masks, const int32_t* tile_offsets,
                                               const int32_t* flatten_ids, int64_t I, int64_t nnz, int32_t channels,
                                               int32_t image_width, int32_t image_height, int32_t tile_size,
                                               int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                               float* render_colors, float* render_alphas, int32_t* last_ids,
                                               void* stream) {
  return rasterize_fwd_impl(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, I, nnz,
                            nnz, channels, image_width, image_height, tile_size, tile_width, tile_height, n_isects,
                            render_colors, render_alphas, last_ids, stream);
}

extern "C" int gsplat_hip_rasterize_bwd(const float* means2d, const float* conics, const float* colors,
                                        const float* opacities, const float* backgrounds, const uint8_t* masks,
                                        const int32_t* tile_offsets, const int32_t* flatten_ids, int64_t I, int64_t N,
                                        int32_t channels, int32_t image_width, int32_t image_height, int32_t tile_size,
                                        int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                        const float* render_alphas, const int32_t* last_ids,
                                        const float* v_render_colors, const float* v_render_alphas,
                                        float* v_means2d_abs, float* v_means2d, float* v_conics, float* v_colors,
                                        float* v_opacities, float* v_backgrounds, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return rasterize_bwd_impl(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, I, N,
                            I * N, channels, image_width, image_height, tile_size, tile_width, tile_height, n_isects,
                            render_alphas, last_ids, v_render_colors, v_render_alphas, v_means2d_abs, v_means2d,
                            v_conics, v_colors, v_opacities, v_backgrounds, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_rasterize_bwd_packed(const float* means2d, const float* conics, const float* colors,
                                               const float* opacities, const float* backgrounds,
                                               const uint8_t* masks, const int32_t* tile_offsets,
                                               const int32_t* flatten_ids, int64_t I, int64_t nnz, int32_t channels,
                                               int32_t image_width, int32_t image_height, int32_t tile_size,
                                               int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                               const float* render_alphas, const int32_t* last_ids,
                                               const float* v_render_colors, const float* v_render_alphas,
                                               float* v_means2d_abs, float* v_means2d, float* v_conics,
                                               float* v_colors, float* v_opacities, float* v_backgrounds,
                                               void* workspace, size_t workspace_bytes, void* stream) {
  return rasterize_bwd_impl(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, I, nnz,
                            nnz, channels, image_width, image_height, tile_size, tile_width, tile_height, n_isects,
                            render_alphas, last_ids, v_render_colors, v_render_alphas, v_means2d_abs, v_means2d,
                            v_conics, v_colors, v_opacities, v_backgrounds, workspace, workspace_bytes, stream);
}

// Device address of `scratch` on the current device, looked up once per
// device (hipGetSymbolAddress with that device current) and kept.
static int noalloc_scratch(void** ptr, const char* what) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> cache[kMaxDevices];
  static std::mutex mu;
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), what);
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices) return invalid(std::string(what) + ": device index out of range.");
  void* p = cache[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(mu);
    p = cache[dev].load(std::memory_order_relaxed);
    if (!p) {
      if ((rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), what))) return rc;
      if (!p) return invalid(std::string(what) + ": no scratch address.");
      cache[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return GSPLAT_OK;
}

extern "C" size_t gsplat_hip_rasterize_bwd_noalloc_max_scratch(void) { return kNoAllocScratchBytes; }

extern "C" int gsplat_hip_rasterize_bwd_noalloc(const float* means2d, const float* conics, const float* colors,
                                                const float* opacities, const float* backgrounds,
                                                const uint8_t* masks, const int32_t* tile_offsets,
                                                const int32_t* flatten_ids, int64_t I, int64_t N, int32_t channels,
                                                int32_t image_width, int32_t image_height, int32_t tile_size,
                                                int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                                const float* render_alphas, const int32_t* last_ids,
                                                const float* v_render_colors, const float* v_render_alphas,
                                                float* v_means2d_abs, float* v_means2d, float* v_conics,
                                                float* v_colors, float* v_opacities, float* v_backgrounds,
                                                void* stream) {
  const char* what = "rasterize_to_pixels_3dgs_backward_noalloc";
  RasterArgs a{means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, N, channels,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects, I * N};
  int rc = check_args(a, what);
  if (rc) return rc;
  const int64_t n_total = I * tile_width * static_cast<int64_t>(tile_height);
  // every schedule word and background partial the kernels read is written
  // earlier in the same call, so nothing in the scratch needs clearing
  if (n_total > 0 && bwd_workspace_bytes(n_total, channels) > kNoAllocScratchBytes)
    return invalid(std::string(what) + ": the tile schedule needs " +
                   std::to_string(bwd_workspace_bytes(n_total, channels)) + " bytes (images * tiles * (8 + 4 * " +
                   "channels), rounded), more than the " + std::to_string(kNoAllocScratchBytes) +
                   "-byte static scratch; use gsplat_hip_rasterize_bwd with a workspace.");
  void* ws = nullptr;
  if ((rc = noalloc_scratch(&ws, what))) return rc;
  return rasterize_bwd_impl(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, I, N,
                            I * N, channels, image_width, image_height, tile_size, tile_width, tile_height, n_isects,
                            render_alphas, last_ids, v_render_colors, v_render_alphas, v_means2d_abs, v_means2d,
                            v_conics, v_colors, v_opacities, v_backgrounds, ws, kNoAllocScratchBytes, stream);
}

static int raster_indices_args(const char* what, const RasterArgs& a) {
  int rc = check_args(a, what);
  if (rc) return rc;
  if (a.ts * a.ts > 1024) return invalid(std::string(what) + ": tile_size must be at most 32.");
  if (a.I > 0 && a.tw > 0 && a.th > 0 && (!a.tile_offsets || (a.n_isects > 0 && !a.flatten_ids)))
    return invalid(std::string(what) + ": null pointer.");
  if (a.n_isects > 0 && (!a.means2d || !a.conics || !a.opacities)) return invalid(std::string(what) + ": null pointer.");
  return GSPLAT_OK;
}

extern "C" size_t gsplat_hip_rasterize_to_indices_workspace_size(int64_t I, int32_t image_width,
                                                                 int32_t image_height) {
  return scan_workspace_bytes(I * image_width * static_cast<int64_t>(image_height));
}

extern "C" int gsplat_hip_rasterize_to_indices_count(int64_t range_start, int64_t range_end,
                                                     const float* transmittances, const float* means2d,
                                                     const float* conics, const float* opacities,
                                                     const int32_t* tile_offsets, const int32_t* flatten_ids,
                                                     int64_t I, int64_t n_rows, int32_t image_width,
                                                     int32_t image_height, int32_t tile_size, int32_t tile_width,
                                                     int32_t tile_height, int64_t n_isects, int32_t* starts,
                                                     int64_t* total_dev, void* workspace, size_t workspace_bytes,
                                                     void* stream) {
  const char* what = "rasterize_to_indices_3dgs";
  RasterArgs a{means2d, conics, nullptr, opacities, nullptr, nullptr, tile_offsets, flatten_ids, n_rows, 1,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects, n_rows};
  int rc = raster_indices_args(what, a);
  if (rc) return rc;
  if (!total_dev) return invalid(std::string(what) + ": null total.");
  hipStream_t s = as_stream(stream);
  const int64_t n_pix = I * image_width * static_cast<int64_t>(image_height);
  if (n_pix == 0 || tile_width == 0 || tile_height == 0) return fill_zero(total_dev, sizeof(int64_t), s);
  if (!starts) return invalid(std::string(what) + ": null pointer.");
  if (!workspace || workspace_bytes < scan_workspace_bytes(n_pix)) {
    set_error(std::string(what) + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  const int bs = (tile_size * tile_size + kWave - 1) / kWave * kWave;
  {
    KernelTimer timer("raster_indices", s);
    raster_indices_kernel<false><<<dim3(tile_width, tile_height, static_cast<unsigned>(I)), bs, 0, s>>>(
        a, range_start, range_end, transmittances, starts, nullptr, 0, nullptr, nullptr);
  }
  if ((rc = check_launch(what))) return rc;
  return scan_exclusive_i32(starts, starts, n_pix, total_dev, workspace, s);
}

extern "C" int gsplat_hip_rasterize_to_indices_write(int64_t range_start, int64_t range_end,
                                                     const float* transmittances, const float* means2d,
                                                     const float* conics, const float* opacities,
                                                     const int32_t* tile_offsets, const int32_t* flatten_ids,
                                                     int64_t I, int64_t n_rows, int32_t image_width,
                                                     int32_t image_height, int32_t tile_size, int32_t tile_width,
                                                     int32_t tile_height, int64_t n_isects, const int32_t* starts,
                                                     int64_t n_out, int32_t* out_gauss_ids, int64_t* out_indices,
                                                     void* stream) {
  const char* what = "rasterize_to_indices_3dgs";
  RasterArgs a{means2d, conics, nullptr, opacities, nullptr, nullptr, tile_offsets, flatten_ids, n_rows, 1,
               image_width, image_height, tile_size, tile_width, tile_height, I, n_isects, n_rows};
  int rc = raster_indices_args(what, a);
  if (rc) return rc;
  if (n_out < 0) return invalid(std::string(what) + ": negative output size.");
  const int64_t n_pix = I * image_width * static_cast<int64_t>(image_height);
  if (n_pix == 0 || tile_width == 0 || tile_height == 0 || n_out == 0) return GSPLAT_OK;
  if (!starts || !out_gauss_ids || !out_indices) return invalid(std::string(what) + ": null pointer.");
  hipStream_t s = as_stream(stream);
  const int bs = (tile_size * tile_size + kWave - 1) / kWave * kWave;
  {
    KernelTimer timer("raster_indices", s);
    raster_indices_kernel<true><<<dim3(tile_width, tile_height, static_cast<unsigned>(I)), bs, 0, s>>>(
        a, range_start, range_end, transmittances, nullptr, starts, n_out, out_gauss_ids, out_indices);
  }
  return check_launch(what);
}

extern "C" size_t gsplat_hip_rasterize_bwd_workspace_size(int64_t I, int32_t channels, int32_t tile_width,
                                                          int32_t tile_height) {
  if (I <= 0 || tile_width <= 0 || tile_height <= 0 || channels <= 0) return 0;
  return bwd_workspace_bytes(I * tile_width * static_cast<int64_t>(tile_height), channels);
}
