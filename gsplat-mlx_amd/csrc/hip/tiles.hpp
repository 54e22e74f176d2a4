// The reference's AABB tile rectangle of a projected Gaussian and the
// ellipse (AccuTile) tiles within it, shared by the intersection pipelines.
#pragma once

#include "common.hpp"

namespace gsplat_hip {

struct TileRect {
  int min_x, min_y, max_x, max_y;  // [min, max) in tile units
};

// v / ts in float. For a power-of-two ts the product with the exact
// reciprocal is the same correctly rounded value (both round v 2^-k), without
// the division sequence; ts is uniform, so the branch is too.
__device__ __forceinline__ float div_tile(float v, int ts) {
  const float fts = static_cast<float>(ts);
  if ((ts & (ts - 1)) == 0) return v * (1.0f / fts);
  return v / fts;
}

// gsplat_intersect.cpp:67-99: float divisions by the tile size, floor / ceil,
// clamped to [0, tw] x [0, th] (the max is exclusive); empty for a zero radius.
__device__ __forceinline__ TileRect aabb_tile_rect(float mx, float my, int rx, int ry, int ts, int tw, int th) {
  TileRect r = {0, 0, 0, 0};
  if (rx <= 0 || ry <= 0) return r;
  const float trx = div_tile(static_cast<float>(rx), ts);
  const float try_ = div_tile(static_cast<float>(ry), ts);
  const float tx = div_tile(mx, ts);
  const float ty = div_tile(my, ts);
  r.min_x = min(max(0, static_cast<int>(floorf(tx - trx))), tw);
  r.min_y = min(max(0, static_cast<int>(floorf(ty - try_))), th);
  r.max_x = min(max(0, static_cast<int>(ceilf(tx + trx))), tw);
  r.max_y = min(max(0, static_cast<int>(ceilf(ty + try_))), th);
  return r;
}

// ---------------------------------------------------------------------------
// Ellipse tile intersection (the use_conics / use_opacities path that
// gsplat_intersect.cpp:123-126 rejects and leaves to upstream gsplat's
// IntersectTile.cu, Task_Metal.md:95-115). The method is Speedy-Splat's
// SnugBox + AccuTile (Hanson et al., CVPR 2025): a Gaussian only needs the
// tiles where some pixel centre can pass the rasterizer's alpha test,
// alpha = min(0.99, o exp(-sigma)) >= 1/255, sigma = d^T Q d / 2 with Q the
// conic. That holds inside the ellipse d^T Q d <= 2 ln(255 o); the test below
// uses the same slack as the rasterizer's per-wave cull, 1.05 ln(255 o) +
// 1e-4, and the same conditions under which a conic is never culled, so
// every entry it drops has alpha < 1/255 at every pixel of the dropped tile.
//
// Tiles are the Gaussian's AABB rect (aabb_tile_rect, the reference set)
// intersected with the ellipse, row by row: within tile row ty the pixel
// centres span y in [ty ts + 1/2, ty ts + ts - 1/2]; the ellipse's x-extent
// over that slab is [xl, xr], where the extreme points of the ellipse
// (dy = -/+ b x_ext / c) are clamped into the slab (the boundary is concave
// on the right and convex on the left, so the clamped point is the extreme);
// the row's tiles are the columns whose pixel centres meet [xl, xr]. Every
// row's tiles are contiguous, and entries keep the reference's order:
// row-major within each Gaussian.
//
// Only + - * /, sqrt, floor and frexp are used, with contraction off, so the
// CPU restatement gives the same tiles bit for bit.
//
// mode 0: no tiles (opacity <= 0, or ln(255 o) too small for any pixel);
// mode 1: the whole rect (non-finite values, opacity NaN or too large for
//         the log, conic not positive-definite or det <= 1e-4 a c);
// mode 2: per-row intervals.
struct EllipseTiles {
  TileRect r;
  int mode;
  float mx, my, a, b, det, aR, ye, dyl;
};

// ln z for finite z > 0: z = m 2^e with m in [sqrt(1/2), sqrt(2)), and
// ln m = 2 atanh(s), s = (m - 1) / (m + 1), |s| < 0.172, by the odd series
// to s^9 (truncation below 1e-9 relative).
__device__ __forceinline__ float ellipse_ln(float z) {
  int e = 0;
  float m = frexpf(z, &e);
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

// One Gaussian's inputs to the tile test (conic and opacity zero when the
// lists are AABB rects).
struct GaussTileIn {
  float mx, my, a, b, c, o;
  int rx, ry;
};

__device__ __forceinline__ GaussTileIn load_gauss_tile_in(const float* __restrict__ means2d,
                                                          const int32_t* __restrict__ radii,
                                                          const float* __restrict__ conics,
                                                          const float* __restrict__ opacities, int64_t g) {
  GaussTileIn in;
  in.mx = means2d[g * 2];
  in.my = means2d[g * 2 + 1];
  in.rx = radii[g * 2];
  in.ry = radii[g * 2 + 1];
  const bool ell = conics && opacities;
  in.a = ell ? conics[g * 3] : 0.0f;
  in.b = ell ? conics[g * 3 + 1] : 0.0f;
  in.c = ell ? conics[g * 3 + 2] : 0.0f;
  in.o = ell ? opacities[g] : 0.0f;
  return in;
}

// ell false: the whole rect (AABB lists).
__device__ __forceinline__ EllipseTiles ellipse_tiles_of(const GaussTileIn& in, bool ell, int ts, int tw, int th) {
  EllipseTiles e;
  e.mx = in.mx;
  e.my = in.my;
  e.r = aabb_tile_rect(e.mx, e.my, in.rx, in.ry, ts, tw, th);
  e.mode = 1;
  e.a = e.b = e.det = e.aR = e.ye = e.dyl = 0.0f;
  if (e.r.max_x <= e.r.min_x || e.r.max_y <= e.r.min_y) {
    e.mode = 0;
    return e;
  }
  if (!ell) return e;  // AABB lists: the whole rect
  const float o = in.o;
  if (o <= 0.0f) {
    e.mode = 0;
    return e;
  }
  const float z = 255.0f * o;
  const float a = in.a, b = in.b, c = in.c;
  if (!(z < 3.0e38f) || !(a > 0.0f && c > 0.0f && a < 1.0e30f && c < 1.0e30f) ||
      !(fabsf(e.mx) < 1.0e30f) || !(fabsf(e.my) < 1.0e30f))
    return e;
  const float det = a * c - b * b;
  if (!(det > 1.0e-4f * a * c)) return e;
  const float lim = 1.05f * ellipse_ln(z) + 1.0e-4f;  // bound on sigma
  if (!(lim >= 0.0f)) {
    e.mode = 0;
    return e;
  }
  const float R = 2.0f * lim;  // bound on d^T Q d
  const float xe = sqrtf(R * c / det);
  e.mode = 2;
  e.a = a;
  e.b = b;
  e.det = det;
  e.aR = a * R;
  e.ye = sqrtf(R * a / det);
  e.dyl = b * xe / c;  // dy of the leftmost point; the rightmost is at -dyl
  // Rows outside [my - ye, my + ye] (with a row of margin either side) are
  // empty: drop them from the rect so that no loop visits them.
  const float ylo = floorf(div_tile(e.my - e.ye, ts)) - 1.0f;
  const float yhi = floorf(div_tile(e.my + e.ye, ts)) + 2.0f;
  const float fy0 = static_cast<float>(e.r.min_y), fy1 = static_cast<float>(e.r.max_y);
  e.r.min_y = static_cast<int>(fminf(fmaxf(ylo, fy0), fy1));
  e.r.max_y = static_cast<int>(fminf(fmaxf(yhi, fy0), fy1));
  return e;
}

__device__ __forceinline__ EllipseTiles ellipse_tiles(const float* __restrict__ means2d,
                                                      const int32_t* __restrict__ radii,
                                                      const float* __restrict__ conics,
                                                      const float* __restrict__ opacities, int64_t g, int ts,
                                                      int tw, int th) {
  return ellipse_tiles_of(load_gauss_tile_in(means2d, radii, conics, opacities, g), conics && opacities, ts, tw,
                          th);
}

// Columns [*c0, *c1) of tile row ty (empty: *c1 <= *c0).
__device__ __forceinline__ void ellipse_row(const EllipseTiles& e, int ty, int ts, int* c0, int* c1) {
  if (e.mode != 2) {
    *c0 = e.r.min_x;
    *c1 = e.mode == 1 ? e.r.max_x : e.r.min_x;
    return;
  }
  const float y0 = static_cast<float>(ty * ts) + 0.5f;
  const float y1 = y0 + static_cast<float>(ts - 1);
  const float d0 = fmaxf(y0 - e.my, -e.ye);
  const float d1 = fminf(y1 - e.my, e.ye);
  if (!(d0 <= d1)) {
    *c0 = *c1 = e.r.min_x;
    return;
  }
  const float dl = fminf(fmaxf(e.dyl, d0), d1);
  const float dr = fminf(fmaxf(-e.dyl, d0), d1);
  const float ql = sqrtf(fmaxf(e.aR - e.det * dl * dl, 0.0f));
  const float qr = sqrtf(fmaxf(e.aR - e.det * dr * dr, 0.0f));
  const float xl = e.mx - (e.b * dl + ql) / e.a;
  const float xr = e.mx + (qr - e.b * dr) / e.a;
  const float lo = floorf(div_tile(xl + 0.5f, ts));
  const float hi = floorf(div_tile(xr - 0.5f, ts)) + 1.0f;
  const float fmin = static_cast<float>(e.r.min_x), fmax = static_cast<float>(e.r.max_x);
  *c0 = static_cast<int>(fminf(fmaxf(lo, fmin), fmax));
  *c1 = static_cast<int>(fminf(fmaxf(hi, fmin), fmax));
}

// Tile of the Gaussian's k-th entry (row-major); false when k is past its
// last entry (offsets inconsistent with the counts).
__device__ __forceinline__ bool ellipse_locate(const EllipseTiles& e, int ts, int k, int* ty, int* tx, int* row_end) {
  for (int y = e.r.min_y; y < e.r.max_y; ++y) {
    int c0, c1;
    ellipse_row(e, y, ts, &c0, &c1);
    const int w = max(c1 - c0, 0);
    if (k < w) {
      *ty = y;
      *tx = c0 + k;
      *row_end = c1;
      return true;
    }
    k -= w;
  }
  return false;
}

}  // namespace gsplat_hip
