// Tile-bucketed intersection for gfx950: the sorted intersection list of
// GSPlatIntersectTile with sort = true (gsplat_intersect.cpp:213-286) without
// a device-wide radix sort.
//
// The reference encodes key = image << (32 + tile_bits) | tile << 32 | depth
// bits Gaussian-major and argsorts it; a stable sort leaves every (image,
// tile) list in ascending (depth bits, flatten id) order. Here:
//  1. grid pass (one block per range of BucketDims::gpb Gaussians of one
//     image): each Gaussian's AABB tile rect adds +1, -1, -1, +1 at its four
//     corners of a (th + 1) x (tw + 1) difference grid in LDS (four LDS
//     atomics per Gaussian whatever its size; ellipse lists: four per tile
//     row of the ellipse, each row a rect one tile high); the block stores
//     its grid, and tiles_per_gauss is written here;
//  2. block scan: per grid point, the exclusive sum of the grids of the
//     image's earlier blocks (in place) and the image total;
//  3. tile pass (one block): the 2D inclusive prefix of an image's total grid
//     is every tile's entry count; their exclusive scan is each tile's first
//     slot (the reference's tile offsets), the total M and the largest count;
//     lists too long for the smallest tile sort are binned by length class;
//     -- the caller reads M and the largest count back --
//  4. scatter (the grid pass's blocks again): each block turns its exclusive
//     grid into per-tile bases by the same 2D prefix in LDS, adds the tile
//     starts, and writes one (depth bits, flatten id) pair per entry at its
//     tile's base plus an LDS counter; the block's entries are dealt evenly
//     over its threads (a Gaussian may cover thousands of tiles; ellipse
//     lists: the entries of the round's tile rows);
//  5. tile sort (one block per tile): the tile's pairs are sorted in LDS by a
//     stable LSD radix sort on the depth bits, 8 bits a pass (passes whose
//     digit is the same for the whole tile are skipped); a tile holding two
//     equal depths is sorted again on (depth bits, flatten id), the id bytes
//     as the low digits, so the order is the reference's whatever order the
//     scatter left; the block writes the 64-bit ids and the flatten ids.
//     Short lists are sorted by one launch over every list, each longer
//     class by a launch of a larger instantiation; lists longer than the
//     LDS holds (kBucketMaxList) are split by their most significant varying
//     depth byte into runs that the LDS sort takes in turn.
// Steps 4-5 need M only to size their outputs, and the longest list (read
// back with M) to launch only the classes present.
//
// Rows: dense inputs hold N Gaussians per image, row image * N + n. Packed
// inputs (one row per visible (image, Gaussian) pair, grouped by image as the
// packed projection writes them) hold the rows of image i at [row_start[i],
// row_start[i + 1]), found on the device from the rows' image ids. Either
// way an image's rows are cut into segments of at most gpb rows, one grid /
// scatter block each, and a row's flatten id is its row index.
#include <algorithm>
#include <string>

#include "tiles.hpp"

namespace gsplat_hip {
namespace {

constexpr int kBucketBlock = 1024;                 // grid and scatter passes
constexpr int kXcds = 8;                           // MI355X: workgroups are dealt round-robin over 8 XCDs
constexpr int kBucketMaxGrid = 35072;              // (th + 1)(tw + 1) words of LDS, at most
constexpr int kColGroup = 64, kColSegs = 16;       // block scan: 64 grid points x 16 block ranges
constexpr int kBucketMaxList = 16384;              // longest list the LDS tile sort holds
constexpr int kTilePassBlock = 1024;

inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

struct BucketDims {
  int64_t I, N, bpi;  // images, Gaussians per image, grid blocks per image (dense)
  int64_t gpb;        // Gaussians per grid / scatter block (a multiple of kBucketBlock)
  int tw, th, ts;
  int64_t G;          // grid words per image, (th + 1)(tw + 1)
  int64_t n_tiles;    // tw * th
  int64_t n_seg;      // grid / scatter blocks: I * bpi (dense), ceil(rows / gpb) + I at most (packed)
  // packed rows (nullptr: dense): [I + 1] first segment and first row of each
  // image, the rows' image ids, and a word set when a row's image id is not
  // its segment's (rows not grouped by image, or ids outside [0, I))
  const int32_t* seg_start;
  const int32_t* row_start;
  const int32_t* image_ids;
  int32_t* ungrouped;
};

// The rows of grid / scatter block lb: image, first row and row count (0 for
// the packed layout's spare blocks past the last segment).
struct Segment {
  int64_t image, row0, rows;
};

__device__ __forceinline__ Segment segment_of(const BucketDims& d, int64_t lb) {
  Segment s;
  if (!d.seg_start) {
    s.image = lb / d.bpi;
    const int64_t n0 = (lb % d.bpi) * d.gpb;
    s.row0 = s.image * d.N + n0;
    s.rows = max<int64_t>(0, min<int64_t>(d.gpb, d.N - n0));
    return s;
  }
  int lo = 0, hi = static_cast<int>(d.I) - 1;  // the last image whose first segment is <= lb
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (d.seg_start[mid] <= lb) lo = mid; else hi = mid - 1;
  }
  s.image = lo;
  s.row0 = d.row_start[lo] + (lb - d.seg_start[lo]) * d.gpb;
  s.rows = max<int64_t>(0, min<int64_t>(d.gpb, d.row_start[lo + 1] - s.row0));
  return s;
}

// Tile sort capacities: lists up to kSortCap[0] take the <256, 10> sort in
// one launch over every list; longer lists are binned by the tile pass into
// classes 0-2 (up to kSortCap[1..3]: <512, 8>, <512, 16>, <1024, 16>), each
// sorted by its own launch, and class 3 (longer than LDS holds) by the split
// sort below. At multiview_3m (lists of up to ~10,000) the tile sort takes
// 2.25 ms this way against 2.78 ms with every list in the instantiation the
// longest list needs; <512, 5> for the short lists and <1024, 8> for class 2
// measured slower.
constexpr int kSortCap[4] = {256 * 10, 512 * 8, 512 * 16, 1024 * 16};
constexpr int kSortClasses = 4;

// count workspace: per-block grids [n_seg][G], image total grids [I][G],
// tile starts [I * n_tiles], the long lists of each class [4][I * n_tiles],
// the class sizes [4] (+ the split sort's fallback count), and for packed
// rows the segment and row starts [I + 1] each and the ungrouped word
struct CountLayout {
  int32_t* partials;
  int32_t* totals;
  int32_t* tile_start;
  int32_t* class_lists;
  int32_t* class_counts;
  int32_t* seg_start;
  int32_t* row_start;
  int32_t* ungrouped;
};

size_t count_layout(const BucketDims& d, CountLayout* l, void* base) {
  const size_t a = align256(static_cast<size_t>(d.n_seg * d.G) * 4);
  const size_t b = align256(static_cast<size_t>(d.I * d.G) * 4);
  const size_t c = align256(static_cast<size_t>(d.I * d.n_tiles) * 4);
  const size_t e = align256(static_cast<size_t>(kSortClasses * d.I * d.n_tiles) * 4);
  const size_t f = align256((kSortClasses + 1) * 4);  // class sizes, then the split sort's fallback count
  const size_t r = align256(static_cast<size_t>(d.I + 1) * 4);  // packed: segment / row starts
  const size_t rows_b = d.bpi == 0 ? 2 * r + align256(4) : 0;
  if (l && base) {
    char* p = static_cast<char*>(base);
    l->partials = reinterpret_cast<int32_t*>(p);
    l->totals = reinterpret_cast<int32_t*>(p + a);
    l->tile_start = reinterpret_cast<int32_t*>(p + a + b);
    l->class_lists = reinterpret_cast<int32_t*>(p + a + b + c);
    l->class_counts = reinterpret_cast<int32_t*>(p + a + b + c + e);
    l->seg_start = rows_b ? reinterpret_cast<int32_t*>(p + a + b + c + e + f) : nullptr;
    l->row_start = rows_b ? reinterpret_cast<int32_t*>(p + a + b + c + e + f + r) : nullptr;
    l->ungrouped = rows_b ? reinterpret_cast<int32_t*>(p + a + b + c + e + f + 2 * r) : nullptr;
  }
  return a + b + c + e + f + rows_b;
}

// Packed rows (one block of kRowsBlock threads): each image's first row as
// the lower bound of its id in the rows' ids (made non-decreasing, so the
// segments stay inside [0, rows) whatever the ids), its segments of at most
// gpb rows, and the ungrouped word cleared -- or set at once when the ids do
// not start at image 0 or end below I.
constexpr int kRowsBlock = 256;

__global__ void __launch_bounds__(kRowsBlock) bucket_rows_kernel(const int32_t* __restrict__ image_ids, int64_t rows,
                                                                 int64_t I, int64_t gpb, int32_t* __restrict__ row_start,
                                                                 int32_t* __restrict__ seg_start,
                                                                 int32_t* __restrict__ ungrouped) {
  const int t = threadIdx.x;
  for (int64_t i = t; i <= I; i += kRowsBlock) {
    int64_t lo = 0, hi = rows;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (image_ids[mid] < i) lo = mid + 1; else hi = mid;
    }
    row_start[i] = static_cast<int32_t>(lo);
  }
  __syncthreads();
  if (t != 0) return;
  const bool bad = row_start[0] != 0 || row_start[I] != rows;
  int32_t prev = 0;
  int64_t seg = 0;
  for (int64_t i = 0; i <= I; ++i) {
    const int32_t r = max(row_start[i], prev);
    row_start[i] = r;
    if (i > 0) seg += (r - prev + gpb - 1) / gpb;
    seg_start[i] = static_cast<int32_t>(seg);
    prev = r;
  }
  *ungrouped = bad ? 1 : 0;
}

// The grid and scatter passes' block b (in dispatch order) takes the
// Gaussian range of logical block L(b): the XCD that receives workgroups x,
// x + 8, x + 16, ... gets a contiguous run of logical blocks, so the per-tile
// bucket ranges of neighbouring blocks, which share cache lines, are written
// through the same L2. A bijection of [0, nb); results do not depend on it.
__device__ __forceinline__ int64_t logical_block(int64_t b, int64_t nb) {
  const int64_t q = nb / kXcds, r = nb % kXcds;
  const int64_t x = b % kXcds, i = b / kXcds;
  return x * q + min(x, r) + i;
}

// Block-wide (blockDim.x == B, a multiple of 64) exclusive scan of one int64
// per thread; returns the prefix and the total (all threads).
template <int B>
__device__ int64_t block_scan_i64(int64_t v, int64_t* total) {
  __shared__ int64_t s_w[B / kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t inc = wave_inclusive_scan_i64(v);
  if (lane == kWave - 1) s_w[wave] = inc;
  __syncthreads();
  int64_t wb = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < B / kWave; ++w) {
    const int64_t x = s_w[w];
    wb += w < wave ? x : 0;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return wb + inc - v;
}

// ---------------------------------------------------------------------------
// Ellipse (AccuTile) tiles: every tile row of a Gaussian's ellipse is a
// contiguous column span [c0, c1) (ellipse_row), so each row is a rect one
// tile high and adds its own four corners to the same difference grid; the
// scatter deals the same rows' entries. Both passes hold the round's
// geometry in LDS, compacted to ten words per Gaussian, and deal the round's
// (Gaussian, row) pairs over the block, kEllRowChunk at a time, one per
// thread (a wave waits for the block's mean row count, not for its largest
// Gaussian): each Gaussian's thread writes its own index and row number into
// the chunk slots of its rows, and the slot's thread computes that row's
// span. The geometry and every row span come from the same code in both
// passes, so the counts and the scatter agree.
struct EllRec {
  float mx, my, a, b, det, aR, ye, dyl;
  uint32_t xs;  // min_x | max_x << 16
  uint32_t ym;  // min_y | mode << 16
};

__device__ __forceinline__ EllRec ell_pack(const EllipseTiles& e) {
  EllRec r;
  r.mx = e.mx;
  r.my = e.my;
  r.a = e.a;
  r.b = e.b;
  r.det = e.det;
  r.aR = e.aR;
  r.ye = e.ye;
  r.dyl = e.dyl;
  r.xs = static_cast<uint32_t>(e.r.min_x) | (static_cast<uint32_t>(e.r.max_x) << 16);
  r.ym = static_cast<uint32_t>(e.r.min_y) | (static_cast<uint32_t>(e.mode) << 16);
  return r;
}

// Row k of the record's rows: its y and its column span.
__device__ __forceinline__ int ell_row(const EllRec& r, int k, int ts, int* c0, int* c1) {
  EllipseTiles e;
  e.mx = r.mx;
  e.my = r.my;
  e.a = r.a;
  e.b = r.b;
  e.det = r.det;
  e.aR = r.aR;
  e.ye = r.ye;
  e.dyl = r.dyl;
  e.r.min_x = static_cast<int>(r.xs & 0xffffu);
  e.r.max_x = static_cast<int>(r.xs >> 16);
  e.r.min_y = static_cast<int>(r.ym & 0xffffu);
  e.r.max_y = 0;  // unused by ellipse_row
  e.mode = static_cast<int>(r.ym >> 16);
  const int y = e.r.min_y + k;
  ellipse_row(e, y, ts, c0, c1);
  return y;
}

constexpr int kEllRowChunk = kBucketBlock;  // tile rows per chunk, one per thread
constexpr int kEllGaussBits = 10;           // round index bits of a chunk slot
static_assert((1 << kEllGaussBits) == kBucketBlock, "chunk slots hold a round index");

// The round's geometry: thread t's Gaussian (inputs `in`, absent when
// !valid) into s_r[t]; *pre, *rows: its first row in the round and its row
// count. Returns the round's rows (block-uniform).
__device__ __forceinline__ int ell_round(const GaussTileIn& in, bool valid, const BucketDims& d, EllRec* s_r,
                                         int* pre, int* rows) {
  EllipseTiles e;
  e.r = {0, 0, 0, 0};
  e.mode = 0;
  e.mx = e.my = e.a = e.b = e.det = e.aR = e.ye = e.dyl = 0.0f;
  *rows = 0;
  if (valid) {
    e = ellipse_tiles_of(in, true, d.ts, d.tw, d.th);
    if (e.mode != 0) *rows = max(e.r.max_y - e.r.min_y, 0);
  }
  s_r[threadIdx.x] = ell_pack(e);
  int64_t tot;
  *pre = static_cast<int>(block_scan_i64<kBucketBlock>(*rows, &tot));  // syncs
  return static_cast<int>(tot);
}

// Thread t's Gaussian of the round (row idx; zeros past the segment): loaded
// one round ahead, so the loads are in flight while the previous round's rows
// are dealt.
__device__ __forceinline__ GaussTileIn ell_load(const float* __restrict__ means2d, const int32_t* __restrict__ radii,
                                                const float* __restrict__ conics,
                                                const float* __restrict__ opacities, int64_t idx, bool valid) {
  GaussTileIn in = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0, 0};
  if (valid) in = load_gauss_tile_in(means2d, radii, conics, opacities, idx);
  return in;
}

// Packed rows: a row whose image id is not its segment's marks the input
// ungrouped (the caller then takes another path; nothing here reads out of
// bounds either way).
__device__ __forceinline__ void check_row_image(const BucketDims& d, int64_t idx, int64_t image) {
  if (d.image_ids && d.image_ids[idx] != image) atomicOr(d.ungrouped, 1);
}

// Slots of chunk [c, c + kEllRowChunk) held by this thread's rows
// [pre, pre + rows): round index | row number << kEllGaussBits.
__device__ __forceinline__ void ell_owners(int c, int pre, int rows, uint32_t* s_own) {
  const int k0 = max(pre, c), k1 = min(pre + rows, c + kEllRowChunk);
  for (int k = k0; k < k1; ++k)
    s_own[k - c] = static_cast<uint32_t>(threadIdx.x) | (static_cast<uint32_t>(k - pre) << kEllGaussBits);
}

constexpr size_t kEllGridLds = kBucketBlock * sizeof(EllRec) + (kEllRowChunk + kBucketBlock) * 4;
constexpr size_t kEllScatterLds = kBucketBlock * sizeof(EllRec) + kBucketBlock * 4 + (4 * kEllRowChunk + 1) * 4;
constexpr size_t kLdsBytes = 160 * 1024;  // MI355X LDS per workgroup
// static LDS beside the dynamic grid: block_scan_i64's per-wave totals
constexpr size_t kBlockScanLds = (kBucketBlock / kWave) * sizeof(int64_t);
constexpr int kBucketMaxGridEll = static_cast<int>((kLdsBytes - kEllScatterLds - kBlockScanLds) / 4);
static_assert(kEllGridLds <= kEllScatterLds, "the ellipse scatter's LDS bounds the ellipse grid pass's");
static_assert(kBucketMaxGrid * 4 + (4 * kBucketBlock + 1) * 4 + kBlockScanLds <= kLdsBytes,
              "the AABB scatter's LDS fits a workgroup");

// ---------------------------------------------------------------------------
// 1. Difference grid of the block's Gaussians' rects (ELL: of their ellipse
// rows).
template <bool ELL>
__global__ void __launch_bounds__(kBucketBlock) bucket_grid_kernel(const float* __restrict__ means2d,
                                                                   const int32_t* __restrict__ radii,
                                                                   const float* __restrict__ conics,
                                                                   const float* __restrict__ opacities, BucketDims d,
                                                                   int32_t* __restrict__ tiles_per_gauss,
                                                                   int32_t* __restrict__ partials) {
  extern __shared__ int32_t sg[];  // [G]; ELL: then the round's records, row prefix and counts
  const int t = threadIdx.x;
  const int64_t lb = logical_block(blockIdx.x, d.n_seg);
  const Segment seg = segment_of(d, lb);
  if (d.seg_start && seg.rows == 0) return;  // a packed spare block: its grid is never read
  const int64_t image = seg.image;
  const int W1 = d.tw + 1;
  for (int j = t; j < d.G; j += kBucketBlock) sg[j] = 0;
  __syncthreads();
  if constexpr (!ELL) {
    for (int64_t i = t; i < seg.rows; i += kBucketBlock) {
      const int64_t idx = seg.row0 + i;
      check_row_image(d, idx, image);
      const TileRect r = aabb_tile_rect(means2d[idx * 2], means2d[idx * 2 + 1], radii[idx * 2], radii[idx * 2 + 1],
                                        d.ts, d.tw, d.th);
      const int area = (r.max_y - r.min_y) * (r.max_x - r.min_x);
      tiles_per_gauss[idx] = area;
      if (area > 0) {
        atomicAdd(&sg[r.min_y * W1 + r.min_x], 1);
        atomicAdd(&sg[r.min_y * W1 + r.max_x], -1);
        atomicAdd(&sg[r.max_y * W1 + r.min_x], -1);
        atomicAdd(&sg[r.max_y * W1 + r.max_x], 1);
      }
    }
  } else {
    EllRec* s_r = reinterpret_cast<EllRec*>(sg + d.G);
    uint32_t* s_own = reinterpret_cast<uint32_t*>(s_r + kBucketBlock);  // [kEllRowChunk] chunk slots
    int32_t* s_cnt = reinterpret_cast<int32_t*>(s_own + kEllRowChunk);  // entries per Gaussian
    GaussTileIn next = ell_load(means2d, radii, conics, opacities, seg.row0 + t, t < seg.rows);
    for (int64_t i0 = 0; i0 < seg.rows; i0 += kBucketBlock) {
      const bool valid = i0 + t < seg.rows;
      const int64_t idx = seg.row0 + i0 + t;
      if (valid) check_row_image(d, idx, image);
      s_cnt[t] = 0;
      int pre, my_rows;
      const int rows = ell_round(next, valid, d, s_r, &pre, &my_rows);  // syncs
      if (i0 + kBucketBlock < seg.rows)
        next = ell_load(means2d, radii, conics, opacities, idx + kBucketBlock, i0 + kBucketBlock + t < seg.rows);
      for (int c = 0; c < rows; c += kEllRowChunk) {
        ell_owners(c, pre, my_rows, s_own);
        __syncthreads();
        if (t < rows - c) {
          const uint32_t v = s_own[t];
          const int gi = static_cast<int>(v & (kBucketBlock - 1));
          int c0, c1;
          const int y = ell_row(s_r[gi], static_cast<int>(v >> kEllGaussBits), d.ts, &c0, &c1);
          if (c1 > c0) {
            atomicAdd(&sg[y * W1 + c0], 1);
            atomicAdd(&sg[y * W1 + c1], -1);
            atomicAdd(&sg[(y + 1) * W1 + c0], -1);
            atomicAdd(&sg[(y + 1) * W1 + c1], 1);
            atomicAdd(&s_cnt[gi], c1 - c0);
          }
        }
        __syncthreads();  // the chunk's slots are rewritten next chunk
      }
      // the last chunk's barrier ordered every count of this round; the next
      // round's block scan orders this read before its slots and counts are
      // written by other threads
      if (valid) tiles_per_gauss[idx] = s_cnt[t];
    }
  }
  __syncthreads();
  int32_t* out = partials + lb * d.G;
  for (int j = t; j < d.G; j += kBucketBlock) out[j] = sg[j];
}

// 2. Per grid point, the exclusive sum over the image's blocks (in place) and
// the image total. Thread (seg, col) sums a contiguous range of blocks for
// grid point col of its group (a wave reads 64 consecutive grid words of one
// block grid); the 16 range sums are scanned in LDS. A range of up to
// kScanRegs blocks (768 blocks per image) is loaded once, all loads in
// flight together, and kept in registers for the write-back.
constexpr int kScanRegs = 48;

__global__ void __launch_bounds__(kColGroup* kColSegs) bucket_block_scan_kernel(BucketDims d,
                                                                                  int32_t* __restrict__ partials,
                                                                                  int32_t* __restrict__ totals) {
  __shared__ int32_t s_sum[kColSegs][kColGroup];
  const int col = threadIdx.x % kColGroup, seg = threadIdx.x / kColGroup;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kColGroup + col;
  const int64_t image = blockIdx.y;
  // the image's blocks: [s0, s0 + nb)
  const int64_t s0 = d.seg_start ? d.seg_start[image] : image * d.bpi;
  const int64_t nb = d.seg_start ? d.seg_start[image + 1] - s0 : d.bpi;
  const int64_t per = (nb + kColSegs - 1) / kColSegs;
  const bool in_regs = per <= kScanRegs;  // uniform
  const int64_t b0 = min<int64_t>(nb, seg * per), b1 = min<int64_t>(nb, b0 + per);
  int32_t* base = partials + s0 * d.G + g;
  int32_t v[kScanRegs];
  int32_t s = 0;
  if (g < d.G) {
    if (in_regs) {
#pragma unroll
      for (int k = 0; k < kScanRegs; ++k) v[k] = b0 + k < b1 ? base[(b0 + k) * d.G] : 0;
#pragma unroll
      for (int k = 0; k < kScanRegs; ++k) s += v[k];
    } else {
      for (int64_t b = b0; b < b1; ++b) s += base[b * d.G];
    }
  }
  s_sum[seg][col] = s;
  __syncthreads();
  int32_t run = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < kColSegs; ++k) {
    const int32_t x = s_sum[k][col];
    run += k < seg ? x : 0;
    tot += x;
  }
  if (g >= d.G) return;
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kScanRegs; ++k) {
      if (b0 + k < b1) base[(b0 + k) * d.G] = run;
      run += v[k];
    }
  } else {
    for (int64_t b = b0; b < b1; ++b) {
      const int32_t x = base[b * d.G];
      base[b * d.G] = run;
      run += x;
    }
  }
  if (seg == 0) totals[image * d.G + g] = tot;
}

// Inclusive prefix of n words at p[0], p[stride], ... by one wave: 64 at a
// time, a DPP scan of each chunk plus the carry of the chunks before.
__device__ __forceinline__ void wave_prefix_strided(int32_t* p, int n, int stride) {
  const int lane = threadIdx.x % kWave;
  int32_t carry = 0;
  for (int c = 0; c < n; c += kWave) {
    const int i = c + lane;
    const int32_t v = wave_inclusive_scan(i < n ? p[i * stride] : 0) + carry;
    if (i < n) p[i * stride] = v;
    carry = __builtin_amdgcn_readlane(v, kWave - 1);
  }
}

// 2D inclusive prefix of a (th + 1) x (tw + 1) grid in LDS: every row, then
// every column, each by one wave (the block's waves take rows / columns in
// turn).
__device__ void grid_prefix_2d(int32_t* g, int tw, int th, int nthreads) {
  const int W1 = tw + 1, H1 = th + 1;
  const int wave = threadIdx.x / kWave, n_waves = nthreads / kWave;
  for (int y = wave; y < H1; y += n_waves) wave_prefix_strided(g + y * W1, W1, 1);
  __syncthreads();
  for (int x = wave; x < W1; x += n_waves) wave_prefix_strided(g + x, H1, W1);
  __syncthreads();
}

// 3. Tile counts, tile starts, M and the largest count (one block; images in
// turn, each grid in LDS); lists longer than kSortCap[0] are appended to their
// sort class's list.
__global__ void __launch_bounds__(kTilePassBlock) bucket_tile_pass_kernel(BucketDims d,
                                                                          const int32_t* __restrict__ totals,
                                                                          int32_t* __restrict__ tile_start,
                                                                          int32_t* __restrict__ class_lists,
                                                                          int32_t* __restrict__ class_counts,
                                                                          int64_t* __restrict__ readback) {
  extern __shared__ int32_t sg[];  // [G]
  __shared__ int32_t s_cls[kSortClasses];
  const int t = threadIdx.x;
  if (t < kSortClasses) s_cls[t] = 0;  // ordered before use by the first image's barrier
  const int64_t n_lists = d.I * d.n_tiles;
  const int W1 = d.tw + 1;
  int64_t offset = 0;  // entries of earlier images
  int32_t largest = 0;
  // thread t: tiles [k0, k1) of each image in row-major order, from tile
  // (x0, y0) (32-bit: an image holds fewer than 2^31 tiles)
  const int n_tiles = static_cast<int>(d.n_tiles);
  const int per = (n_tiles + kTilePassBlock - 1) / kTilePassBlock;
  const int k0 = min(n_tiles, t * per), k1 = min(n_tiles, k0 + per);
  const int y0 = k0 / d.tw, x0 = k0 - y0 * d.tw;
  for (int64_t image = 0; image < d.I; ++image) {
    for (int j = t; j < d.G; j += kTilePassBlock) sg[j] = totals[image * d.G + j];
    __syncthreads();
    grid_prefix_2d(sg, d.tw, d.th, kTilePassBlock);
    int64_t sum = 0;
    for (int k = k0, x = x0, y = y0; k < k1; ++k) {
      const int32_t c = sg[y * W1 + x];
      sum += c;
      largest = max(largest, c);
      if (++x == d.tw) {
        x = 0;
        ++y;
      }
    }
    int64_t tot;
    int64_t run = offset + block_scan_i64<kTilePassBlock>(sum, &tot);
    int32_t* starts = tile_start + image * d.n_tiles;
    for (int k = k0, x = x0, y = y0; k < k1; ++k) {
      starts[k] = static_cast<int32_t>(run);
      const int32_t c = sg[y * W1 + x];
      run += c;
      if (c > kSortCap[0]) {  // rare: a long list goes to its class
        const int cls = c <= kSortCap[1] ? 0 : (c <= kSortCap[2] ? 1 : (c <= kSortCap[3] ? 2 : 3));
        class_lists[cls * n_lists + atomicAdd(&s_cls[cls], 1)] = static_cast<int32_t>(image * d.n_tiles + k);
      }
      if (++x == d.tw) {
        x = 0;
        ++y;
      }
    }
    offset += tot;
    __syncthreads();  // sg is reloaded for the next image
  }
  // the largest count over all threads
  __shared__ int32_t s_max[kTilePassBlock / kWave];
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) largest = max(largest, __shfl_xor(largest, off, kWave));
  if (t % kWave == 0) s_max[t / kWave] = largest;
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kTilePassBlock / kWave; ++w) largest = max(largest, s_max[w]);
    readback[0] = offset;
    readback[1] = largest;
    if (d.ungrouped) readback[2] = *d.ungrouped;
  }
  if (t <= kSortClasses) class_counts[t] = t < kSortClasses ? s_cls[t] : 0;  // + the fallback count
}

// 4. Scatter of the (depth bits, flatten id) pairs into the tile buckets.
//
// The round's entries are dealt evenly over the block's threads: thread t
// writes entries [e0, e1) of the round's `units` (rects: origin s_xy = min x
// | min y << 16, entry prefix s_pre[0..n_units]; s_w the width, and the
// unit is Gaussian u of the round; ROWS: s_w = width | Gaussian << 16),
// row-major within each unit, eight at a time (their tiles, then their
// eight LDS cursor increments, then their eight stores, so the round trips
// overlap); the current unit's record stays in registers.
template <bool ROWS>
__device__ __forceinline__ void scatter_units(int64_t tot, int n_units, const int32_t* s_pre, const uint32_t* s_xy,
                                              const int32_t* s_w, const uint32_t* s_d,
                                              uint32_t id0, int W1, int32_t* sg, int64_t n_isects,
                                              uint2* __restrict__ pairs) {
  const int t = threadIdx.x;
  const int64_t e0 = tot * t / kBucketBlock, e1 = tot * (t + 1) / kBucketBlock;
  if (e0 >= e1) return;
  // the unit holding entry e0: the last one whose prefix is <= e0
  int lo = 0, hi = n_units - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pre[mid] <= e0) lo = mid; else hi = mid - 1;
  }
  int u = lo;
  int next = s_pre[u + 1], w = ROWS ? (s_w[u] & 0xffff) : s_w[u], gi = ROWS ? (s_w[u] >> 16) : u;
  uint32_t xy = s_xy[u];
  const int local = static_cast<int>(e0 - s_pre[u]);
  int row = local / w, col = local - row * w;
  constexpr int kBatch = 8;
  for (int64_t e = e0; e < e1;) {
    int ci[kBatch], gg[kBatch];
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (e + k >= e1) break;
      while (e + k >= next) {  // past this unit's entries (empty units are skipped)
        ++u;
        next = s_pre[u + 1];
        w = ROWS ? (s_w[u] & 0xffff) : s_w[u];
        xy = s_xy[u];
        gi = ROWS ? (s_w[u] >> 16) : u;
        row = 0;
        col = 0;
      }
      ci[k] = (static_cast<int>(xy >> 16) + row) * W1 + static_cast<int>(xy & 0xffffu) + col;
      gg[k] = gi;
      if (++col == w) {
        col = 0;
        ++row;
      }
      cnt = k + 1;
    }
    int pos[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (k < cnt) pos[k] = atomicAdd(&sg[ci[k]], 1);
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (k < cnt && pos[k] < n_isects)  // always, for the counts of the same inputs
        pairs[pos[k]] = make_uint2(s_d[gg[k]], id0 + static_cast<uint32_t>(gg[k]));
    e += cnt;
  }
}

// AABB (ELL false): the units are the round's Gaussians' rects. ELL: the
// units are the round's ellipse tile rows (rects one tile high), taken
// kEllRowChunk at a time.
template <bool ELL>
__global__ void __launch_bounds__(kBucketBlock) bucket_scatter_kernel(const float* __restrict__ means2d,
                                                                      const int32_t* __restrict__ radii,
                                                                      const float* __restrict__ conics,
                                                                      const float* __restrict__ opacities,
                                                                      const float* __restrict__ depths, BucketDims d,
                                                                      const int32_t* __restrict__ partials,
                                                                      const int32_t* __restrict__ tile_start,
                                                                      int64_t n_isects, uint2* __restrict__ pairs) {
  extern __shared__ int32_t sg[];  // [G] per-tile cursors, then the round's records
  const int t = threadIdx.x;
  const int64_t lb = logical_block(blockIdx.x, d.n_seg);
  const Segment seg = segment_of(d, lb);
  if (d.seg_start && seg.rows == 0) return;  // a packed spare block
  const int64_t image = seg.image;
  const int W1 = d.tw + 1;
  const int32_t* ex = partials + lb * d.G;
  for (int j = t; j < d.G; j += kBucketBlock) sg[j] = ex[j];
  __syncthreads();
  grid_prefix_2d(sg, d.tw, d.th, kBucketBlock);
  // entries of earlier blocks + the tile's first slot
  for (int j = t; j < d.G; j += kBucketBlock) {
    const int y = j / W1, x = j % W1;
    if (y < d.th && x < d.tw) sg[j] += tile_start[image * d.n_tiles + y * d.tw + x];
  }
  __syncthreads();
  if constexpr (!ELL) {
    int32_t* s_pre = sg + d.G;                                           // [kBucketBlock + 1] entry prefix
    uint32_t* s_xy = reinterpret_cast<uint32_t*>(s_pre + kBucketBlock + 1);  // rect min x | min y << 16
    int32_t* s_w = reinterpret_cast<int32_t*>(s_xy + kBucketBlock);          // rect width
    uint32_t* s_d = reinterpret_cast<uint32_t*>(s_w + kBucketBlock);         // depth bits
    for (int64_t i0 = 0; i0 < seg.rows; i0 += kBucketBlock) {
      int area = 0;
      if (i0 + t < seg.rows) {
        const int64_t idx = seg.row0 + i0 + t;
        const TileRect r = aabb_tile_rect(means2d[idx * 2], means2d[idx * 2 + 1], radii[idx * 2],
                                          radii[idx * 2 + 1], d.ts, d.tw, d.th);
        area = (r.max_y - r.min_y) * (r.max_x - r.min_x);
        s_xy[t] = static_cast<uint32_t>(r.min_x) | (static_cast<uint32_t>(r.min_y) << 16);
        s_w[t] = r.max_x - r.min_x;
        s_d[t] = __float_as_uint(depths[idx]);
      }
      int64_t tot;
      const int64_t pre = block_scan_i64<kBucketBlock>(area, &tot);
      s_pre[t] = static_cast<int32_t>(pre);
      if (t == 0) s_pre[kBucketBlock] = static_cast<int32_t>(tot);
      __syncthreads();
      const uint32_t id0 = static_cast<uint32_t>(seg.row0 + i0);
      scatter_units<false>(tot, kBucketBlock, s_pre, s_xy, s_w, s_d, id0, W1, sg, n_isects, pairs);
      __syncthreads();  // the round's LDS records are rewritten next round
    }
  } else {
    EllRec* s_r = reinterpret_cast<EllRec*>(sg + d.G);
    uint32_t* s_d = reinterpret_cast<uint32_t*>(s_r + kBucketBlock);         // depth bits
    uint32_t* s_own = s_d + kBucketBlock;                                     // [kEllRowChunk] chunk slots
    int32_t* s_epre = reinterpret_cast<int32_t*>(s_own + kEllRowChunk);      // [kEllRowChunk + 1] entry prefix
    uint32_t* s_xy = reinterpret_cast<uint32_t*>(s_epre + kEllRowChunk + 1);  // row c0 | y << 16
    int32_t* s_w = reinterpret_cast<int32_t*>(s_xy + kEllRowChunk);          // row width | Gaussian << 16
    GaussTileIn next = ell_load(means2d, radii, conics, opacities, seg.row0 + t, t < seg.rows);
    for (int64_t i0 = 0; i0 < seg.rows; i0 += kBucketBlock) {
      const bool valid = i0 + t < seg.rows;
      const int64_t idx = seg.row0 + i0 + t;
      if (valid) s_d[t] = __float_as_uint(depths[idx]);
      int pre, my_rows;
      const int rows = ell_round(next, valid, d, s_r, &pre, &my_rows);  // syncs
      if (i0 + kBucketBlock < seg.rows)
        next = ell_load(means2d, radii, conics, opacities, idx + kBucketBlock, i0 + kBucketBlock + t < seg.rows);
      const uint32_t id0 = static_cast<uint32_t>(seg.row0 + i0);
      for (int c = 0; c < rows; c += kEllRowChunk) {
        const int nr = min(kEllRowChunk, rows - c);
        ell_owners(c, pre, my_rows, s_own);
        __syncthreads();
        int w = 0;
        if (t < nr) {
          const uint32_t v = s_own[t];
          const int gi = static_cast<int>(v & (kBucketBlock - 1));
          int c0, c1;
          const int y = ell_row(s_r[gi], static_cast<int>(v >> kEllGaussBits), d.ts, &c0, &c1);
          w = max(c1 - c0, 0);
          s_xy[t] = static_cast<uint32_t>(c0) | (static_cast<uint32_t>(y) << 16);
          // an empty row is skipped by its prefix; width 1 keeps the walk's division defined
          s_w[t] = max(w, 1) | (gi << 16);
        }
        int64_t tot;
        const int64_t epre = block_scan_i64<kBucketBlock>(w, &tot);  // syncs
        if (t < nr) s_epre[t] = static_cast<int32_t>(epre);
        if (t == 0) s_epre[nr] = static_cast<int32_t>(tot);
        __syncthreads();
        scatter_units<true>(tot, nr, s_epre, s_xy, s_w, s_d, id0, W1, sg, n_isects, pairs);
        __syncthreads();  // the chunk's rows are rewritten next chunk
      }
      // s_d and s_r are rewritten next round only after the last chunk's barrier
    }
  }
}

// 5. Tile sort. Elements live in LDS in list order; wave w holds the
// contiguous chunk [w R 64, (w + 1) R 64) in registers, R = ceil(n / (W 64))
// rounds of 64, so every wave holds part of even a short list. One stable
// pass on an 8-bit digit: wave-private running digit counts rank each wave's
// chunk (ballots, as the device-wide sort), the per-digit counts are scanned
// over waves and digits, and the elements are written back to LDS in digit
// order. A pass whose digit is one value for the whole list is skipped.
// Each element is one 8-byte LDS word (depth bits, flatten id), so a pass
// reads and scatters it with one instruction.
template <int B, int ITEMS>
struct TileSorter {
  static constexpr int W = B / kWave;
  static constexpr int CAP = B * ITEMS;
  uint2* kv;          // [CAP] (depth bits, flatten id)
  uint32_t* wcnt;     // [W][256]
  uint32_t* dstart;   // [256]
  int n, R;

  // sorts on byte `shift / 8` of the depth bits (by_id false) or of the ids;
  // vary: the bits of that byte that differ between elements (none: the pass
  // is the identity and is skipped)
  __device__ void pass(bool by_id, int shift, uint32_t vary) {
    if (vary == 0) return;  // block-uniform
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    uint32_t k[ITEMS], v[ITEMS], rank[ITEMS];
    for (int j = t; j < W * 256; j += B) wcnt[j] = 0;
    __syncthreads();
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    uint32_t* wc = wcnt + wave * 256;
    // fully unrolled, so k, v and rank stay in registers (a runtime index
    // would put them in scratch memory)
#pragma clang loop unroll(full)
    for (int r = 0; r < ITEMS; ++r) {
      if (r >= R) break;  // wave-uniform
      const int idx = (wave * R + r) * kWave + lane;
      const bool valid = idx < n;
      const uint2 e = valid ? kv[idx] : make_uint2(0u, 0u);
      k[r] = e.x;
      v[r] = e.y;
      const uint32_t dg = ((by_id ? v[r] : k[r]) >> shift) & 255u;
      // lanes with the same digit: for each bit, ballot the lanes whose bit is
      // clear and keep the ballot (or its complement) that contains this lane;
      // z = 0 / ~0 for a set / clear bit, so ~(ballot ^ z) holds this lane
      // (one v_bitop3 per half)
      const uint64_t vm = __ballot(valid);
      uint32_t plo = static_cast<uint32_t>(vm), phi = static_cast<uint32_t>(vm >> 32);
      const uint32_t nd = ~dg;
      // all eight bits, unrolled: skipping the bits every element shares
      // (uniform branches, or a scalar loop over the varying bits) measured
      // slower, and with 16 items the branches put the arrays in scratch
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const int32_t x = static_cast<int32_t>(nd << (31 - b));
        const uint32_t z = static_cast<uint32_t>(x >> 31);
        const uint64_t m = __ballot(x < 0);
        plo &= ~(static_cast<uint32_t>(m) ^ z);
        phi &= ~(static_cast<uint32_t>(m >> 32) ^ z);
      }
      const uint64_t peers = (static_cast<uint64_t>(phi) << 32) | plo;
      const uint32_t my = static_cast<uint32_t>(__popcll(peers & below));
      const uint32_t cur = valid ? wc[dg] : 0u;
      rank[r] = cur + my;
      if (valid && my == 0) wc[dg] = cur + static_cast<uint32_t>(__popcll(peers));
    }
    __syncthreads();
    if (t < 256) {
      uint32_t run = 0;
      for (int w = 0; w < W; ++w) {
        const uint32_t c = wcnt[w * 256 + t];
        wcnt[w * 256 + t] = run;
        run += c;
      }
      dstart[t] = run;
    }
    __syncthreads();
    if (t < kWave) {  // exclusive scan of the 256 digit totals, 4 per lane
      uint32_t c[4];
      uint32_t s = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = dstart[t * 4 + q];
        s += c[q];
      }
      const uint32_t inc = static_cast<uint32_t>(wave_inclusive_scan(static_cast<int>(s)));  // wave 0, all lanes
      uint32_t run = inc - s;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        dstart[t * 4 + q] = run;
        run += c[q];
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
      if (r >= R) break;
      const int idx = (wave * R + r) * kWave + lane;
      if (idx < n) {
        const uint32_t dg = ((by_id ? v[r] : k[r]) >> shift) & 255u;
        const uint32_t pos = dstart[dg] + wcnt[wave * 256 + dg] + rank[r];
        kv[pos] = make_uint2(k[r], v[r]);
      }
    }
    __syncthreads();
  }
};

// The n (depth bits, flatten id) pairs at src sorted in LDS (the shared
// arrays of the calling kernel) and written as ids hi | depth bits and
// flatten ids at out_ids / out_flat. Every input is read before any output
// is written, so src may be the bytes of out_ids. n > CAP is left alone.
template <int B, int ITEMS>
__device__ __forceinline__ void sort_range(const uint2* src, int64_t len, uint64_t hi, int64_t* out_ids,
                                           int32_t* out_flat, uint2* s_kv,
                                           uint32_t* s_wcnt, uint32_t* s_dstart, uint32_t* s_bits) {
  using S = TileSorter<B, ITEMS>;
  if (len <= 0 || len > S::CAP) return;  // block-uniform
  const int n = static_cast<int>(len);
  const int t = threadIdx.x;
  if (t < 4) s_bits[t] = (t & 1) ? ~0u : 0u;
  __syncthreads();
  // the bits that vary over the list: passes on digits every element shares
  // are skipped. The list is loaded ITEMS elements per thread, all loads in
  // flight before the first LDS store (lists this sort holds have at most
  // B * ITEMS elements).
  uint32_t ko = 0u, ka = ~0u, vo = 0u, va = ~0u;
  {
    uint2 e[ITEMS];
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
      const int j = r * B + t;
      e[r] = j < n ? src[j] : make_uint2(0u, ~0u);
    }
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
      const int j = r * B + t;
      if (j < n) {
        s_kv[j] = e[r];
        ko |= e[r].x;
        ka &= e[r].x;
        vo |= e[r].y;
        va &= e[r].y;
      }
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    ko |= __shfl_xor(ko, off, kWave);
    ka &= __shfl_xor(ka, off, kWave);
    vo |= __shfl_xor(vo, off, kWave);
    va &= __shfl_xor(va, off, kWave);
  }
  if (t % kWave == 0) {
    atomicOr(&s_bits[0], ko);
    atomicAnd(&s_bits[1], ka);
    atomicOr(&s_bits[2], vo);
    atomicAnd(&s_bits[3], va);
  }
  __syncthreads();
  const uint32_t kvary = s_bits[0] ^ s_bits[1], ivary = s_bits[2] ^ s_bits[3];
  S srt{s_kv, s_wcnt, s_dstart, n, (n + S::W * kWave - 1) / (S::W * kWave)};
  if (n > 1) {
#pragma unroll 1
    for (int shift = 0; shift < 32; shift += 8) srt.pass(false, shift, (kvary >> shift) & 255u);
    // equal depths: their entries go in flatten-id order. A run of up to
    // kShortRun equal keys is insertion-sorted by the thread at its start;
    // a list with a longer run is sorted again, ids as the low digits.
    constexpr int kShortRun = 32;
    auto run_start = [&](int j) {
      return j + 1 < n && s_kv[j + 1].x == s_kv[j].x && (j == 0 || s_kv[j - 1].x != s_kv[j].x);
    };
    auto run_end = [&](int j) {
      int e = j + 1;
      while (e < n && s_kv[e].x == s_kv[j].x && e - j <= kShortRun) ++e;
      return e;
    };
    bool tie = false, long_run = false;
    for (int j = t; j < n; j += B) {
      if (run_start(j)) {
        tie = true;
        long_run = long_run || run_end(j) - j > kShortRun;
      }
    }
    const bool any_long = __syncthreads_or(long_run);
    if (any_long) {
#pragma unroll 1
      for (int shift = 0; shift < 32; shift += 8) srt.pass(true, shift, (ivary >> shift) & 255u);
#pragma unroll 1
      for (int shift = 0; shift < 32; shift += 8) srt.pass(false, shift, (kvary >> shift) & 255u);
    } else if (__syncthreads_or(tie)) {
      for (int j = t; j < n; j += B) {
        if (!run_start(j)) continue;
        const int e = run_end(j);
        for (int a = j + 1; a < e; ++a) {  // insertion sort of the ids of [j, e)
          const uint32_t v = s_kv[a].y;
          int b = a - 1;
          while (b >= j && s_kv[b].y > v) {
            s_kv[b + 1].y = s_kv[b].y;
            --b;
          }
          s_kv[b + 1].y = v;
        }
      }
      __syncthreads();
    }
  }
  // every thread read its inputs before the first barrier above
  for (int j = t; j < n; j += B) {
    const uint2 e = s_kv[j];
    out_ids[j] = static_cast<int64_t>(hi | e.x);
    out_flat[j] = static_cast<int32_t>(e.y);
  }
}

// The 64-bit id prefix image << (32 + tile_bits) | tile << 32 of list `list`.
__device__ __forceinline__ uint64_t list_hi(int64_t list, int64_t n_tiles, int tile_bits) {
  const int64_t image = list / n_tiles, tile = list % n_tiles;
  return (static_cast<uint64_t>(image) << (32 + tile_bits)) | (static_cast<uint64_t>(tile) << 32);
}

// [*start, *end) of tile list `list` (clamped to [0, n_isects]).
__device__ __forceinline__ void list_range(int64_t list, const int32_t* __restrict__ tile_start, int64_t n_lists,
                                           int64_t n_isects, int64_t* start, int64_t* end) {
  *end = min<int64_t>(list + 1 < n_lists ? tile_start[list + 1] : n_isects, n_isects);
  *start = min<int64_t>(max<int64_t>(tile_start[list], 0), *end);
}

// One tile list sorted in LDS (the shared arrays of its kernel); a list
// longer than this instantiation holds is left alone.
template <int B, int ITEMS>
__device__ __forceinline__ void sort_tile_list(int64_t list, const uint2* __restrict__ pairs,
                                               const int32_t* __restrict__ tile_start, int64_t n_lists,
                                               int64_t n_isects, int64_t n_tiles, int tile_bits,
                                               int64_t* __restrict__ isect_ids, int32_t* __restrict__ flatten_ids,
                                               uint2* s_kv, uint32_t* s_wcnt,
                                               uint32_t* s_dstart, uint32_t* s_bits) {
  int64_t start, end;
  list_range(list, tile_start, n_lists, n_isects, &start, &end);
  sort_range<B, ITEMS>(pairs + start, end - start, list_hi(list, n_tiles, tile_bits), isect_ids + start,
                       flatten_ids + start, s_kv, s_wcnt, s_dstart, s_bits);
}

template <int B, int ITEMS>
struct TileSortLds {
  using S = TileSorter<B, ITEMS>;
  uint2 kv[S::CAP];
  uint32_t wcnt[S::W * 256];
  uint32_t dstart[256];
  uint32_t bits[4];  // OR and AND of the keys, OR and AND of the ids
};

// Block b sorts list b and writes its tile offset (every list; lists longer
// than this instantiation holds are left to the class kernels).
template <int B, int ITEMS>
__global__ void __launch_bounds__(B) bucket_tile_sort_kernel(const uint2* __restrict__ pairs,
                                                             const int32_t* __restrict__ tile_start, int64_t n_lists,
                                                             int64_t n_isects, const int64_t* __restrict__ m_dev,
                                                             int64_t n_tiles, int tile_bits,
                                                             int64_t* __restrict__ isect_ids,
                                                             int32_t* __restrict__ flatten_ids,
                                                             int32_t* __restrict__ tile_offsets) {
  __shared__ TileSortLds<B, ITEMS> sh;
  if (m_dev) n_isects = min(n_isects, *m_dev);
  const int64_t list = blockIdx.x;
  if (tile_offsets && threadIdx.x == 0) tile_offsets[list] = tile_start[list];
  sort_tile_list<B, ITEMS>(list, pairs, tile_start, n_lists, n_isects, n_tiles, tile_bits, isect_ids, flatten_ids,
                           sh.kv, sh.wcnt, sh.dstart, sh.bits);
}

// Block b sorts list b of one long class (the tile pass's binning); blocks
// past the class's size exit at once.
template <int B, int ITEMS>
__global__ void __launch_bounds__(B) bucket_tile_sort_class_kernel(const uint2* __restrict__ pairs,
                                                                   const int32_t* __restrict__ tile_start,
                                                                   int64_t n_lists, int64_t n_isects,
                                                                   const int64_t* __restrict__ m_dev, int64_t n_tiles,
                                                                   int tile_bits, int64_t* __restrict__ isect_ids,
                                                                   int32_t* __restrict__ flatten_ids,
                                                                   const int32_t* __restrict__ class_list,
                                                                   const int32_t* __restrict__ class_count) {
  __shared__ TileSortLds<B, ITEMS> sh;
  if (static_cast<int>(blockIdx.x) >= *class_count) return;
  if (m_dev) n_isects = min(n_isects, *m_dev);
  sort_tile_list<B, ITEMS>(class_list[blockIdx.x], pairs, tile_start, n_lists, n_isects, n_tiles, tile_bits,
                           isect_ids, flatten_ids, sh.kv, sh.wcnt, sh.dstart, sh.bits);
}

// Lists longer than the LDS sorts hold (class 3). One block per list takes
// the eight bits of the depth keys below and at their most significant
// varying bit as a digit (the keys agree on every higher bit, so every key
// of one digit is smaller than every key of the next) and counts the 256
// digits; when no digit holds more than kRunCap entries, it scatters the
// list by digit into the bytes of its isect_ids, groups consecutive digits
// into runs of at most kRunCap entries, and sorts the runs one after another
// with the LDS sort, which writes the final ids in place. Otherwise (every
// depth equal, or one digit too crowded) the list goes to a block that sorts
// it in global memory: a stable LSD radix sort with the list's pairs and the
// same bytes of its isect_ids as the two buffers, each pass walking the list
// in tiles of kHugeTile entries, wave w ranking its contiguous chunk by
// ballots as TileSorter does; ties of depth are resolved by sorting again on
// the flatten ids, then on the depth bits.
constexpr int kHugeBlock = 1024;
constexpr int kHugeItems = 8;
constexpr int kHugeTile = kHugeBlock * kHugeItems;
constexpr int kHugeWaves = kHugeBlock / kWave;

struct HugeRadixLds {
  uint32_t hist[8][256];  // digit counts: depth bytes 0-3, id bytes 0-3
  uint32_t run[256];      // running start of each digit in the destination
  uint32_t wcnt[kHugeWaves][256];
};

__device__ void huge_hist(const uint2* __restrict__ src, int n, bool ids, HugeRadixLds& sh) {
  const int t = threadIdx.x;
  uint32_t(*h)[256] = sh.hist + (ids ? 4 : 0);
  for (int j = t; j < 4 * 256; j += kHugeBlock) h[j / 256][j % 256] = 0u;
  __syncthreads();
  for (int j = t; j < n; j += kHugeBlock) {
    const uint2 p = src[j];
    const uint32_t v = ids ? p.y : p.x;
#pragma unroll
    for (int q = 0; q < 4; ++q) atomicAdd(&h[q][(v >> (8 * q)) & 255u], 1u);
  }
  __syncthreads();
}

// Exclusive scan of 256 digit counts into `out` by wave 0 (4 digits per
// lane); returns nothing, callers sync.
__device__ __forceinline__ void digit_starts(const uint32_t* counts, uint32_t* out) {
  const int t = threadIdx.x;
  if (t < kWave) {
    uint32_t c[4];
    uint32_t s = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c[q] = counts[t * 4 + q];
      s += c[q];
    }
    const uint32_t inc = static_cast<uint32_t>(wave_inclusive_scan(static_cast<int>(s)));
    uint32_t r = inc - s;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      out[t * 4 + q] = r;
      r += c[q];
    }
  }
}

// One stable pass on byte `shift / 8` of the depth bits (or of the ids) from
// src to dst; hist: that byte's digit counts over the list.
__device__ void huge_pass(const uint2* __restrict__ src, uint2* __restrict__ dst, int n, bool by_id, int shift,
                          const uint32_t* hist, HugeRadixLds& sh) {
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  digit_starts(hist, sh.run);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  uint32_t* wc = sh.wcnt[wave];
  for (int base = 0; base < n; base += kHugeTile) {
    for (int j = t; j < kHugeWaves * 256; j += kHugeBlock) (&sh.wcnt[0][0])[j] = 0u;
    __syncthreads();
    uint2 e[kHugeItems];
    uint32_t rank[kHugeItems];
#pragma unroll
    for (int r = 0; r < kHugeItems; ++r) {
      const int idx = base + (wave * kHugeItems + r) * kWave + lane;
      const bool valid = idx < n;
      e[r] = valid ? src[idx] : make_uint2(0u, 0u);
      const uint32_t dg = ((by_id ? e[r].y : e[r].x) >> shift) & 255u;
      const uint64_t vm = __ballot(valid);
      uint32_t plo = static_cast<uint32_t>(vm), phi = static_cast<uint32_t>(vm >> 32);
      const uint32_t nd = ~dg;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const int32_t x = static_cast<int32_t>(nd << (31 - b));
        const uint32_t z = static_cast<uint32_t>(x >> 31);
        const uint64_t m = __ballot(x < 0);
        plo &= ~(static_cast<uint32_t>(m) ^ z);
        phi &= ~(static_cast<uint32_t>(m >> 32) ^ z);
      }
      const uint64_t peers = (static_cast<uint64_t>(phi) << 32) | plo;
      const uint32_t my = static_cast<uint32_t>(__popcll(peers & below));
      const uint32_t cur = valid ? wc[dg] : 0u;
      rank[r] = cur + my;
      if (valid && my == 0) wc[dg] = cur + static_cast<uint32_t>(__popcll(peers));
    }
    __syncthreads();
    if (t < 256) {  // the tile's digit starts per wave, and the running starts past the tile
      uint32_t run = sh.run[t];
      for (int w = 0; w < kHugeWaves; ++w) {
        const uint32_t c = sh.wcnt[w][t];
        sh.wcnt[w][t] = run;
        run += c;
      }
      sh.run[t] = run;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kHugeItems; ++r) {
      const int idx = base + (wave * kHugeItems + r) * kWave + lane;
      if (idx < n) {
        const uint32_t dg = ((by_id ? e[r].y : e[r].x) >> shift) & 255u;
        dst[wc[dg] + rank[r]] = e[r];
      }
    }
    __syncthreads();  // the destination is complete before it is read; wcnt is cleared next tile
  }
}

// The radix path for one list (a at the pairs, b at its isect_ids' bytes).
__device__ void huge_radix(uint2* a, uint2* b, int n, uint32_t kvary, uint32_t ivary, uint64_t hi,
                           int64_t* out_ids, int32_t* out_flat, HugeRadixLds& sh) {
  const int t = threadIdx.x;
  huge_hist(a, n, false, sh);
  uint2* cur = a;
  uint2* oth = b;
  for (int q = 0; q < 4; ++q)
    if ((kvary >> (8 * q)) & 255u) {
      huge_pass(cur, oth, n, false, 8 * q, sh.hist[q], sh);
      uint2* s = cur;
      cur = oth;
      oth = s;
    }
  bool tie = false;
  for (int j = t; j + 1 < n; j += kHugeBlock) tie = tie || cur[j].x == cur[j + 1].x;
  if (__syncthreads_or(tie)) {  // equal depths: ids as the low digits, then the depth bits again
    huge_hist(cur, n, true, sh);
    for (int q = 0; q < 4; ++q)
      if ((ivary >> (8 * q)) & 255u) {
        huge_pass(cur, oth, n, true, 8 * q, sh.hist[4 + q], sh);
        uint2* s = cur;
        cur = oth;
        oth = s;
      }
    for (int q = 0; q < 4; ++q)
      if ((kvary >> (8 * q)) & 255u) {
        huge_pass(cur, oth, n, false, 8 * q, sh.hist[q], sh);
        uint2* s = cur;
        cur = oth;
        oth = s;
      }
  }
  // when the result lies in the ids' bytes, each entry is read and then
  // overwritten by its own thread
  for (int j = t; j < n; j += kHugeBlock) {
    const uint2 p = cur[j];
    out_flat[j] = static_cast<int32_t>(p.y);
    out_ids[j] = static_cast<int64_t>(hi | p.x);
  }
}

// Split path (one block per class-3 list); lists it cannot split are
// appended to the end of the class-3 array (fallback count class_counts[4]) for
// bucket_huge_radix_kernel.
__global__ void __launch_bounds__(kHugeBlock) bucket_huge_sort_kernel(uint2* __restrict__ pairs,
                                                                      const int32_t* __restrict__ tile_start,
                                                                      int64_t n_lists, int64_t n_isects,
                                                                      const int64_t* __restrict__ m_dev,
                                                                      int64_t n_tiles, int tile_bits,
                                                                      int64_t* __restrict__ isect_ids,
                                                                      int32_t* __restrict__ flatten_ids,
                                                                      int32_t* __restrict__ class_list,
                                                                      int32_t* __restrict__ class_counts) {
  constexpr int kRunItems = 8;
  constexpr int kRunCap = kHugeBlock * kRunItems;
  __shared__ TileSortLds<kHugeBlock, kRunItems> sh;
  __shared__ uint32_t s_hist[256], s_cur[256], s_bits[3];
  __shared__ int32_t s_run[257];
  __shared__ int s_nrun;
  if (m_dev) n_isects = min(n_isects, *m_dev);
  const int t = threadIdx.x;
  const int cnt = class_counts[3];
  for (int li = blockIdx.x; li < cnt; li += gridDim.x) {
    const int64_t list = class_list[li];
    int64_t start, end;
    list_range(list, tile_start, n_lists, n_isects, &start, &end);
    const int n = static_cast<int>(end - start);
    const uint64_t hi = list_hi(list, n_tiles, tile_bits);
    const uint2* a = pairs + start;
    uint2* b = reinterpret_cast<uint2*>(isect_ids + start);
    if (t < 3) s_bits[t] = t == 1 ? ~0u : 0u;
    if (t < 256) s_hist[t] = 0u;
    __syncthreads();
    uint32_t ko = 0u, ka = ~0u;
    for (int j = t; j < n; j += kHugeBlock) {
      const uint32_t k = a[j].x;
      ko |= k;
      ka &= k;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      ko |= __shfl_xor(ko, off, kWave);
      ka &= __shfl_xor(ka, off, kWave);
    }
    if (t % kWave == 0) {
      atomicOr(&s_bits[0], ko);
      atomicAnd(&s_bits[1], ka);
    }
    __syncthreads();
    const uint32_t kvary = s_bits[0] ^ s_bits[1];
    // the digit: the eight key bits at and below the most significant varying bit
    const int shift = kvary == 0u ? 0 : max(31 - __builtin_clz(kvary) - 7, 0);
    for (int j = t; j < n; j += kHugeBlock) atomicAdd(&s_hist[(a[j].x >> shift) & 255u], 1u);
    __syncthreads();
    if (t < 256 && s_hist[t] > static_cast<uint32_t>(kRunCap)) atomicOr(&s_bits[2], 1u);
    digit_starts(s_hist, s_cur);
    __syncthreads();
    if (kvary == 0u || s_bits[2] != 0u) {  // block-uniform: the radix kernel takes it
      if (t == 0) class_list[n_lists - 1 - atomicAdd(&class_counts[4], 1)] = static_cast<int32_t>(list);
      __syncthreads();  // s_bits and the histogram are reset by the next list
      continue;
    }
    if (t == 0) {  // consecutive digits grouped into runs of at most kRunCap entries
      int nr = 0;
      uint32_t acc = 0;
      s_run[0] = 0;
      for (int dg = 0; dg < 256; ++dg) {
        const uint32_t c = s_hist[dg];
        if (acc + c > static_cast<uint32_t>(kRunCap)) {
          s_run[++nr] = static_cast<int32_t>(s_cur[dg]);
          acc = 0;
        }
        acc += c;
      }
      s_run[++nr] = n;
      s_nrun = nr;
    }
    __syncthreads();
    for (int j = t; j < n; j += kHugeBlock) {
      const uint2 p = a[j];
      b[atomicAdd(&s_cur[(p.x >> shift) & 255u], 1u)] = p;
    }
    __syncthreads();
    const int nrun = s_nrun;
    for (int r = 0; r < nrun; ++r) {
      const int r0 = s_run[r], r1 = s_run[r + 1];
      sort_range<kHugeBlock, kRunItems>(b + r0, r1 - r0, hi, isect_ids + start + r0, flatten_ids + start + r0,
                                        sh.kv, sh.wcnt, sh.dstart, sh.bits);
      __syncthreads();  // the sort's LDS is reused by the next run
    }
  }
}

// Radix path for the lists the split path left (every depth equal, or one
// digit with more entries than a run holds).
__global__ void __launch_bounds__(kHugeBlock) bucket_huge_radix_kernel(uint2* __restrict__ pairs,
                                                                       const int32_t* __restrict__ tile_start,
                                                                       int64_t n_lists, int64_t n_isects,
                                                                       const int64_t* __restrict__ m_dev,
                                                                       int64_t n_tiles, int tile_bits,
                                                                       int64_t* __restrict__ isect_ids,
                                                                       int32_t* __restrict__ flatten_ids,
                                                                       const int32_t* __restrict__ class_list,
                                                                       const int32_t* __restrict__ class_counts) {
  __shared__ HugeRadixLds sh;
  __shared__ uint32_t s_bits[4];
  if (m_dev) n_isects = min(n_isects, *m_dev);
  const int t = threadIdx.x;
  const int cnt = class_counts[4];
  for (int li = blockIdx.x; li < cnt; li += gridDim.x) {
    const int64_t list = class_list[n_lists - 1 - li];
    int64_t start, end;
    list_range(list, tile_start, n_lists, n_isects, &start, &end);
    const int n = static_cast<int>(end - start);
    uint2* a = pairs + start;
    uint2* b = reinterpret_cast<uint2*>(isect_ids + start);
    if (t < 4) s_bits[t] = (t & 1) ? ~0u : 0u;
    __syncthreads();
    uint32_t ko = 0u, ka = ~0u, vo = 0u, va = ~0u;
    for (int j = t; j < n; j += kHugeBlock) {
      const uint2 p = a[j];
      ko |= p.x;
      ka &= p.x;
      vo |= p.y;
      va &= p.y;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      ko |= __shfl_xor(ko, off, kWave);
      ka &= __shfl_xor(ka, off, kWave);
      vo |= __shfl_xor(vo, off, kWave);
      va &= __shfl_xor(va, off, kWave);
    }
    if (t % kWave == 0) {
      atomicOr(&s_bits[0], ko);
      atomicAnd(&s_bits[1], ka);
      atomicOr(&s_bits[2], vo);
      atomicAnd(&s_bits[3], va);
    }
    __syncthreads();
    huge_radix(a, b, n, s_bits[0] ^ s_bits[1], s_bits[2] ^ s_bits[3], list_hi(list, n_tiles, tile_bits),
               isect_ids + start, flatten_ids + start, sh);
    __syncthreads();  // LDS is reused by the block's next list
  }
}

// packed: numel rows of I images (grouped by image), segments found on the
// device; otherwise numel = I * N.
int bucket_dims(const char* what, int64_t I, int64_t numel, int32_t ts, int32_t tw, int32_t th, bool ell,
                BucketDims* d, bool packed = false) {
  if (I <= 0 || numel < 0 || ts <= 0 || tw <= 0 || th <= 0 || (!packed && numel % I != 0))
    return invalid(std::string(what) + ": invalid sizes.");
  if (packed && (numel > INT32_MAX || I > INT32_MAX - 1)) return invalid(std::string(what) + ": invalid sizes.");
  if (tw >= 65535 || th >= 65535) return invalid(std::string(what) + ": tile grid too large.");
  *d = BucketDims{};
  d->I = I;
  d->N = packed ? 0 : numel / I;
  // about two grid / scatter blocks per CU of a 256-CU MI355X: the nearest
  // whole number of rounds of kBucketBlock Gaussians (at least one, at most
  // 16); rounding up would leave 1.2 blocks per CU at 640K rows
  const int64_t want = (numel + 511) / 512;
  d->gpb = std::min<int64_t>(16, std::max<int64_t>(1, (want + kBucketBlock / 2) / kBucketBlock)) * kBucketBlock;
  d->bpi = packed ? 0 : std::max<int64_t>(1, (d->N + d->gpb - 1) / d->gpb);
  d->n_seg = packed ? (numel + d->gpb - 1) / d->gpb + I : I * d->bpi;
  d->tw = tw;
  d->th = th;
  d->ts = ts;
  d->G = static_cast<int64_t>(tw + 1) * (th + 1);
  d->n_tiles = static_cast<int64_t>(tw) * th;
  if (d->G > (ell ? kBucketMaxGridEll : kBucketMaxGrid))
    return invalid(std::string(what) + ": tile grid larger than the bucketed intersection supports.");
  if (d->n_seg > kMaxGridX || I * d->n_tiles > INT32_MAX) return invalid(std::string(what) + ": too many tiles.");
  return GSPLAT_OK;
}

// The packed rows' tables in the count workspace (after count_layout).
void attach_rows(BucketDims* d, const CountLayout& l, const int32_t* image_ids) {
  d->seg_start = l.seg_start;
  d->row_start = l.row_start;
  d->image_ids = image_ids;
  d->ungrouped = l.ungrouped;
}

int tile_bits_of(int64_t I, int tw, int th, int* tile_bits) {
  auto fl2 = [](int64_t v) { int b = 0; while ((int64_t{1} << (b + 1)) <= v) ++b; return b + 1; };
  *tile_bits = fl2(static_cast<int64_t>(tw) * th);
  if (*tile_bits + fl2(I) > 32) return invalid("intersect_tile_encode image id and tile id require more than 32 bits.");
  return GSPLAT_OK;
}

bool grid_supported(int64_t I, int32_t tw, int32_t th, int64_t max_grid) {
  return I > 0 && tw > 0 && th > 0 && tw < 65535 && th < 65535 && static_cast<int64_t>(tw + 1) * (th + 1) <= max_grid;
}

// Counts (steps 1-3); ell: ellipse tiles of conics / opacities; packed:
// numel rows with their image_ids (totals_dev then takes a third word, the
// ungrouped flag).
int bucket_count(bool ell, const float* means2d, const int32_t* radii, const float* conics, const float* opacities,
                 bool packed, const int32_t* image_ids, int64_t I, int64_t numel, int32_t tile_size,
                 int32_t tile_width, int32_t tile_height, int32_t* tiles_per_gauss, int64_t* totals_dev,
                 void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "intersect_tile";
  BucketDims d;
  int rc = bucket_dims(what, I, numel, tile_size, tile_width, tile_height, ell, &d, packed);
  if (rc) return rc;
  CountLayout l;
  if (!workspace || workspace_bytes < count_layout(d, &l, workspace)) {
    set_error(std::string(what) + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  if (!totals_dev || (numel > 0 && (!means2d || !radii || !tiles_per_gauss || (ell && (!conics || !opacities)) ||
                                    (packed && !image_ids))))
    return invalid(std::string(what) + ": null pointer.");
  hipStream_t s = as_stream(stream);
  const size_t grid_lds = static_cast<size_t>(d.G) * 4;
  const unsigned blocks = static_cast<unsigned>(d.n_seg);
  if (packed) {
    attach_rows(&d, l, image_ids);
    KernelTimer timer("isect_bucket_grid", s);
    bucket_rows_kernel<<<1, kRowsBlock, 0, s>>>(image_ids, numel, I, d.gpb, l.row_start, l.seg_start, l.ungrouped);
  }
  {
    KernelTimer timer("isect_bucket_grid", s);
    if (ell)
      bucket_grid_kernel<true><<<blocks, kBucketBlock, grid_lds + kEllGridLds, s>>>(
          means2d, radii, conics, opacities, d, tiles_per_gauss, l.partials);
    else
      bucket_grid_kernel<false><<<blocks, kBucketBlock, grid_lds, s>>>(means2d, radii, nullptr, nullptr, d,
                                                                       tiles_per_gauss, l.partials);
  }
  if ((rc = check_launch(what))) return rc;
  {
    KernelTimer timer("isect_bucket_scan", s);
    bucket_block_scan_kernel<<<dim3(static_cast<unsigned>((d.G + kColGroup - 1) / kColGroup),
                                    static_cast<unsigned>(I)),
                               kColGroup * kColSegs, 0, s>>>(d, l.partials, l.totals);
    bucket_tile_pass_kernel<<<1, kTilePassBlock, grid_lds, s>>>(d, l.totals, l.tile_start, l.class_lists,
                                                                 l.class_counts, totals_dev);
  }
  return check_launch(what);
}

// Scatter + tile sort (steps 4-5); ell, packed and image_ids as bucket_count's.
// m_dev (nullable): the device word of the count step's M; n_isects is then
// the outputs' capacity (launched before M is on the host), and every write
// stays below it.
int bucket_sort(bool ell, const float* means2d, const int32_t* radii, const float* conics, const float* opacities,
                const float* depths, bool packed, const int32_t* image_ids, int64_t I, int64_t numel, int32_t tile_size,
                int32_t tile_width, int32_t tile_height, int64_t n_isects, int64_t max_list, int64_t* isect_ids,
                int32_t* flatten_ids, int32_t* tile_offsets, const void* count_workspace, size_t count_workspace_bytes,
                void* workspace, size_t workspace_bytes, void* stream, const int64_t* m_dev = nullptr) {
  const char* what = "intersect_tile";
  BucketDims d;
  int rc = bucket_dims(what, I, numel, tile_size, tile_width, tile_height, ell, &d, packed);
  if (rc) return rc;
  int tile_bits = 0;
  if ((rc = tile_bits_of(I, tile_width, tile_height, &tile_bits))) return rc;
  if (n_isects < 0 || n_isects > INT32_MAX) return invalid(std::string(what) + ": invalid intersection count.");
  if (max_list < 0 || max_list > n_isects) return invalid(std::string(what) + ": invalid longest list.");
  CountLayout l;
  if (!count_workspace || count_workspace_bytes < count_layout(d, &l, const_cast<void*>(count_workspace))) {
    set_error(std::string(what) + ": count workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  if (packed) attach_rows(&d, l, image_ids);
  hipStream_t s = as_stream(stream);
  if (n_isects == 0 && !tile_offsets) return GSPLAT_OK;
  if (n_isects > 0 && (!workspace || workspace_bytes < gsplat_hip_isect_bucket_sort_workspace_size(n_isects))) {
    set_error(std::string(what) + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  if (n_isects > 0 && (!means2d || !radii || !depths || !isect_ids || !flatten_ids || (ell && (!conics || !opacities)) ||
                       (packed && !image_ids)))
    return invalid(std::string(what) + ": null pointer.");
  uint2* pairs = static_cast<uint2*>(workspace);
  if (n_isects > 0) {
    KernelTimer timer("isect_bucket_scatter", s);
    const unsigned blocks = static_cast<unsigned>(d.n_seg);
    const size_t grid_lds = static_cast<size_t>(d.G) * 4;
    const size_t lds = grid_lds + (kBucketBlock + 1 + 3 * kBucketBlock) * 4;
    if (ell)
      bucket_scatter_kernel<true><<<blocks, kBucketBlock, grid_lds + kEllScatterLds, s>>>(
          means2d, radii, conics, opacities, depths, d, l.partials, l.tile_start, n_isects, pairs);
    else
      bucket_scatter_kernel<false><<<blocks, kBucketBlock, lds, s>>>(means2d, radii, nullptr, nullptr, depths, d,
                                                                   l.partials, l.tile_start, n_isects, pairs);
  }
  if ((rc = check_launch(what))) return rc;
  const int64_t n_lists = I * d.n_tiles;
  {
    KernelTimer timer("isect_bucket_tile_sort", s);
    const unsigned grid = static_cast<unsigned>(n_lists);
    // every list up to kSortCap[0] (and every tile offset) in one launch;
    // longer lists by their class, one launch per class present
    bucket_tile_sort_kernel<256, 10><<<grid, 256, 0, s>>>(pairs, l.tile_start, n_lists, n_isects, m_dev,
                                                           d.n_tiles, tile_bits, isect_ids, flatten_ids, tile_offsets);
    // a block per list of the class at most: every list of class k holds
    // more than kSortCap[k - 1] entries, so at most n_isects / (kSortCap[k - 1]
    // + 1) of them exist; blocks past the class's size exit at once
    auto cgrid = [&](int k) {
      return static_cast<unsigned>(std::min<int64_t>(n_lists, n_isects / (kSortCap[k - 1] + 1)));
    };
    if (max_list > kSortCap[0])
      bucket_tile_sort_class_kernel<512, 8><<<cgrid(1), 512, 0, s>>>(pairs, l.tile_start, n_lists, n_isects, m_dev,
                                                                      d.n_tiles, tile_bits, isect_ids, flatten_ids,
                                                                      l.class_lists, l.class_counts);
    if (max_list > kSortCap[1])
      bucket_tile_sort_class_kernel<512, 16><<<cgrid(2), 512, 0, s>>>(
          pairs, l.tile_start, n_lists, n_isects, m_dev, d.n_tiles, tile_bits, isect_ids, flatten_ids,
          l.class_lists + n_lists, l.class_counts + 1);
    if (max_list > kSortCap[2])
      bucket_tile_sort_class_kernel<1024, 16><<<cgrid(3), 1024, 0, s>>>(
          pairs, l.tile_start, n_lists, n_isects, m_dev, d.n_tiles, tile_bits, isect_ids, flatten_ids,
          l.class_lists + 2 * n_lists, l.class_counts + 2);
    if (max_list > kSortCap[3]) {  // lists longer than LDS holds: a block each, taking the lists in turn
      const unsigned hg = std::min(static_cast<unsigned>(n_isects / (kSortCap[3] + 1)), 2048u);
      bucket_huge_sort_kernel<<<hg, kHugeBlock, 0, s>>>(pairs, l.tile_start, n_lists, n_isects, m_dev, d.n_tiles,
                                                         tile_bits, isect_ids, flatten_ids,
                                                         l.class_lists + 3 * n_lists, l.class_counts);
      bucket_huge_radix_kernel<<<hg, kHugeBlock, 0, s>>>(pairs, l.tile_start, n_lists, n_isects, m_dev, d.n_tiles,
                                                          tile_bits, isect_ids, flatten_ids,
                                                          l.class_lists + 3 * n_lists, l.class_counts);
    }
  }
  return check_launch(what);
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" int gsplat_hip_isect_bucket_supported(int64_t I, int32_t tile_width, int32_t tile_height) {
  return grid_supported(I, tile_width, tile_height, kBucketMaxGrid);
}

extern "C" int gsplat_hip_isect_bucket_accutile_supported(int64_t I, int32_t tile_width, int32_t tile_height) {
  return grid_supported(I, tile_width, tile_height, kBucketMaxGridEll);
}

extern "C" int64_t gsplat_hip_isect_bucket_max_list(void) { return kBucketMaxList; }

extern "C" size_t gsplat_hip_isect_bucket_count_workspace_size(int64_t I, int64_t numel, int32_t tile_size,
                                                               int32_t tile_width, int32_t tile_height) {
  BucketDims d;
  if (bucket_dims("intersect_tile", I, numel, tile_size, tile_width, tile_height, false, &d)) return 0;
  return count_layout(d, nullptr, nullptr);
}

extern "C" int gsplat_hip_isect_bucket_count(const float* means2d, const int32_t* radii, int64_t I, int64_t numel,
                                             int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                             int32_t* tiles_per_gauss, int64_t* totals_dev, void* workspace,
                                             size_t workspace_bytes, void* stream) {
  return bucket_count(false, means2d, radii, nullptr, nullptr, false, nullptr, I, numel, tile_size, tile_width, tile_height,
                      tiles_per_gauss, totals_dev, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_isect_bucket_count_accutile(const float* means2d, const int32_t* radii,
                                                      const float* conics, const float* opacities, int64_t I,
                                                      int64_t numel, int32_t tile_size, int32_t tile_width,
                                                      int32_t tile_height, int32_t* tiles_per_gauss,
                                                      int64_t* totals_dev, void* workspace, size_t workspace_bytes,
                                                      void* stream) {
  return bucket_count(true, means2d, radii, conics, opacities, false, nullptr, I, numel, tile_size, tile_width, tile_height,
                      tiles_per_gauss, totals_dev, workspace, workspace_bytes, stream);
}

extern "C" size_t gsplat_hip_isect_bucket_sort_workspace_size(int64_t n_isects) {
  return n_isects <= 0 ? 0 : align256(static_cast<size_t>(n_isects) * sizeof(uint2));
}

extern "C" int gsplat_hip_isect_bucket_sort(const float* means2d, const int32_t* radii, const float* depths,
                                            int64_t I, int64_t numel, int32_t tile_size, int32_t tile_width,
                                            int32_t tile_height, int64_t n_isects, int64_t max_list,
                                            int64_t* isect_ids, int32_t* flatten_ids, int32_t* tile_offsets,
                                            const void* count_workspace, size_t count_workspace_bytes,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  return bucket_sort(false, means2d, radii, nullptr, nullptr, depths, false, nullptr, I, numel, tile_size, tile_width,
                     tile_height, n_isects, max_list, isect_ids, flatten_ids, tile_offsets, count_workspace,
                     count_workspace_bytes, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_isect_bucket_sort_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                                     const float* opacities, const float* depths, int64_t I,
                                                     int64_t numel, int32_t tile_size, int32_t tile_width,
                                                     int32_t tile_height, int64_t n_isects, int64_t max_list,
                                                     int64_t* isect_ids, int32_t* flatten_ids, int32_t* tile_offsets,
                                                     const void* count_workspace, size_t count_workspace_bytes,
                                                     void* workspace, size_t workspace_bytes, void* stream) {
  return bucket_sort(true, means2d, radii, conics, opacities, depths, false, nullptr, I, numel, tile_size, tile_width,
                     tile_height, n_isects, max_list, isect_ids, flatten_ids, tile_offsets, count_workspace,
                     count_workspace_bytes, workspace, workspace_bytes, stream);
}

extern "C" size_t gsplat_hip_isect_bucket_count_packed_workspace_size(int64_t I, int64_t nnz, int32_t tile_size,
                                                                      int32_t tile_width, int32_t tile_height) {
  BucketDims d;
  if (bucket_dims("intersect_tile", I, nnz, tile_size, tile_width, tile_height, false, &d, true)) return 0;
  return count_layout(d, nullptr, nullptr);
}

extern "C" int gsplat_hip_isect_bucket_count_packed(const float* means2d, const int32_t* radii, const float* conics,
                                                    const float* opacities, const int32_t* image_ids, int64_t I,
                                                    int64_t nnz, int32_t tile_size, int32_t tile_width,
                                                    int32_t tile_height, int32_t* tiles_per_gauss,
                                                    int64_t* totals_dev, void* workspace, size_t workspace_bytes,
                                                    void* stream) {
  return bucket_count(conics != nullptr, means2d, radii, conics, opacities, true, image_ids, I, nnz, tile_size, tile_width,
                      tile_height, tiles_per_gauss, totals_dev, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_isect_bucket_sort_packed(const float* means2d, const int32_t* radii, const float* conics,
                                                   const float* opacities, const float* depths,
                                                   const int32_t* image_ids, int64_t I, int64_t nnz,
                                                   int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                                   int64_t n_isects, int64_t max_list, int64_t* isect_ids,
                                                   int32_t* flatten_ids, int32_t* tile_offsets,
                                                   const void* count_workspace, size_t count_workspace_bytes,
                                                   void* workspace, size_t workspace_bytes, void* stream) {
  return bucket_sort(conics != nullptr, means2d, radii, conics, opacities, depths, true, image_ids, I, nnz, tile_size, tile_width, tile_height, n_isects, max_list, isect_ids, flatten_ids, tile_offsets,
                     count_workspace, count_workspace_bytes, workspace, workspace_bytes, stream);
}

// 0, 1, 2, 3 or 4: the tile sort classes beyond the short-list sort that a
// bucket sort launched with this longest list runs.
int class_launches(int64_t max_list) {
  int k = 0;
  while (k < kSortClasses && max_list > kSortCap[k]) ++k;
  return k;
}

extern "C" int gsplat_hip_isect_bucket_sort_covers(int64_t max_list_launched, int64_t longest) {
  return class_launches(longest) <= class_launches(max_list_launched);
}

extern "C" int gsplat_hip_isect_bucket_sort_speculative(
    const float* means2d, const int32_t* radii, const float* conics, const float* opacities, const float* depths,
    int32_t packed, const int32_t* image_ids, int64_t I, int64_t numel, int32_t tile_size, int32_t tile_width,
    int32_t tile_height, int64_t capacity, int64_t max_list, const int64_t* totals_dev, int64_t* isect_ids,
    int32_t* flatten_ids, int32_t* tile_offsets, const void* count_workspace, size_t count_workspace_bytes,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (!totals_dev || capacity <= 0) return invalid("intersect_tile: invalid speculative sort arguments.");
  return bucket_sort(conics != nullptr, means2d, radii, conics, opacities, depths, packed != 0, image_ids, I, numel,
                     tile_size, tile_width, tile_height, capacity, max_list, isect_ids, flatten_ids, tile_offsets,
                     count_workspace, count_workspace_bytes, workspace, workspace_bytes, stream, totals_dev);
}
