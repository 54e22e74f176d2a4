// Tile intersection for gfx950: count + exclusive scan, encode (AABB rect or
// ellipse tiles; dense or packed layout), depth-presorted sort, and tile
// offsets.
//
// Integer semantics follow gsplat_core/gsplat_intersect.cpp:60-112 (rect and
// key layout), :309-339 (count), :433-485 (encode order) and :605-641
// (offsets = lower_bound). Tile ids are bit-exact with the reference: the rect
// uses the same float divisions, floor/ceil and clamps.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <string>

#include "radix_sort.hpp"
#include "scan.hpp"
#include "tiles.hpp"

namespace gsplat_hip {
namespace {

// Ellipse tile geometry (EllipseTiles, ellipse_tiles, ellipse_row,
// ellipse_locate): tiles.hpp, shared with the tile-bucket pipeline.

// Ellipse counts fused with the block-local exclusive scan. The row loops
// are balanced over the block: in each of kScanItems rounds the block's 256
// Gaussians put their geometry in LDS, their row counts are scanned, and the
// threads take the (Gaussian, row) pairs in turn, adding each row's width to
// its Gaussian's count with an LDS atomic. A wave then waits for the block's
// mean row count, not for its largest Gaussian.
__global__ void __launch_bounds__(kScanBlock) count_scan_ellipse_kernel(const float* __restrict__ means2d,
                                                                        const int32_t* __restrict__ radii,
                                                                        const float* __restrict__ conics,
                                                                        const float* __restrict__ opacities,
                                                                        int64_t n, int ts, int tw, int th,
                                                                        int32_t* __restrict__ counts,
                                                                        int32_t* __restrict__ offsets,
                                                                        int64_t* __restrict__ block_sums) {
  __shared__ EllipseTiles s_e[kScanBlock];
  __shared__ int32_t s_pre[kScanBlock];  // exclusive prefix of the row counts
  __shared__ int32_t s_cnt[kScanTile];
  const int t = threadIdx.x;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int k = 0; k < kScanItems; ++k) {
    const int li = k * kScanBlock + t;  // coalesced: consecutive threads, consecutive Gaussians
    const int64_t i = base + li;
    EllipseTiles e = {};
    int rows = 0, direct = 0;
    if (i < n) {
      e = ellipse_tiles(means2d, radii, conics, opacities, i, ts, tw, th);
      if (e.mode == 1) direct = (e.r.max_y - e.r.min_y) * (e.r.max_x - e.r.min_x);
      if (e.mode == 2) rows = max(e.r.max_y - e.r.min_y, 0);
    }
    s_e[t] = e;
    s_cnt[li] = direct;
    int64_t total_rows;
    const int pre = static_cast<int>(block_exclusive_scan(rows, &total_rows));  // syncs
    s_pre[t] = pre;
    __syncthreads();
    for (int u = t; u < static_cast<int>(total_rows); u += kScanBlock) {
      int lo = 0, hi = kScanBlock - 1;  // last owner o with s_pre[o] <= u
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_pre[mid] <= u)
          lo = mid;
        else
          hi = mid - 1;
      }
      const EllipseTiles& eo = s_e[lo];
      int c0, c1;
      ellipse_row(eo, eo.r.min_y + (u - s_pre[lo]), ts, &c0, &c1);
      if (c1 > c0) atomicAdd(&s_cnt[k * kScanBlock + lo], c1 - c0);
    }
    __syncthreads();
  }
  const int64_t tb = base + static_cast<int64_t>(t) * kScanItems;
  int32_t v[kScanItems];
  int64_t sum = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    v[k] = tb + k < n ? s_cnt[t * kScanItems + k] : 0;
    if (tb + k < n) counts[tb + k] = v[k];
    sum += v[k];
  }
  int64_t total;
  int64_t run = block_exclusive_scan(sum, &total);
  if (offsets) {
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
      if (tb + k < n) offsets[tb + k] = static_cast<int32_t>(run);
      run += v[k];
    }
  }
  if (t == 0) block_sums[blockIdx.x] = total;
}

// Count per Gaussian fused with the block-local exclusive scan.
__global__ void __launch_bounds__(kScanBlock) count_scan_local_kernel(const float* __restrict__ means2d,
                                                                      const int32_t* __restrict__ radii,
                                                                      int64_t n, int ts, int tw, int th,
                                                                      int32_t* __restrict__ counts,
                                                                      int32_t* __restrict__ offsets,
                                                                      int64_t* __restrict__ block_sums) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + static_cast<int64_t>(threadIdx.x) * kScanItems;
  int32_t v[kScanItems];
  int64_t sum = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    int32_t c = 0;
    if (i < n) {
      const TileRect r = aabb_tile_rect(means2d[i * 2], means2d[i * 2 + 1], radii[i * 2], radii[i * 2 + 1], ts, tw, th);
      c = (r.max_y - r.min_y) * (r.max_x - r.min_x);
      counts[i] = c;
    }
    v[k] = c;
    sum += c;
  }
  int64_t total;
  int64_t run = block_exclusive_scan(sum, &total);
  if (offsets) {  // null: the caller needs only the counts and their total
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
      if (base + k < n) offsets[base + k] = static_cast<int32_t>(run);
      run += v[k];
    }
  }
  if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

__global__ void __launch_bounds__(kScanBlock) block_sums_scan_kernel(int64_t* __restrict__ sums, int64_t nb,
                                                                    int64_t* __restrict__ total_dev) {
  int64_t carry = 0;
  for (int64_t start = 0; start < nb; start += kScanBlock) {
    const int64_t i = start + threadIdx.x;
    const int64_t v = i < nb ? sums[i] : 0;
    int64_t tot;
    const int64_t ex = block_exclusive_scan(v, &tot);
    if (i < nb) sums[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) *total_dev = carry;
}

__global__ void __launch_bounds__(kScanBlock) add_block_prefix_kernel(int32_t* __restrict__ offsets, int64_t n,
                                                                     const int64_t* __restrict__ sums) {
  const int64_t add = sums[blockIdx.x];
  if (add == 0) return;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int k = threadIdx.x; k < kScanTile; k += kScanBlock) {
    const int64_t i = base + k;
    if (i < n) offsets[i] = static_cast<int32_t>(offsets[i] + add);
  }
}

// Load-balanced encode: a block owns kEncodeG consecutive Gaussians and their
// contiguous output range; each output slot finds its Gaussian by binary
// search over the LDS copy of the offsets, so consecutive lanes write
// consecutive keys (coalesced) however unequal the per-Gaussian counts are.
constexpr int kEncodeBlock = 256;
constexpr int kEncodeG = 256;

__global__ void __launch_bounds__(kEncodeBlock) encode_kernel(const float* __restrict__ means2d,
                                                             const int32_t* __restrict__ radii,
                                                             const float* __restrict__ depths,
                                                             const int32_t* __restrict__ offsets, int64_t numel,
                                                             int64_t n_per_image, int ts, int tw, int th,
                                                             int tile_bits, int64_t n_isects,
                                                             int64_t* __restrict__ isect_ids,
                                                             int32_t* __restrict__ flatten_ids) {
  __shared__ int32_t s_off[kEncodeG];
  __shared__ int32_t s_minx[kEncodeG];
  __shared__ int32_t s_miny[kEncodeG];
  __shared__ int32_t s_w[kEncodeG];
  __shared__ int64_t s_hi[kEncodeG];  // image/tile-row independent high key part: image << (32 + tile_bits)
  __shared__ uint32_t s_bits[kEncodeG];
  __shared__ int64_t s_end;
  const int64_t g0 = static_cast<int64_t>(blockIdx.x) * kEncodeG;
  const int cnt = static_cast<int>(min<int64_t>(kEncodeG, numel - g0));
  const int t = threadIdx.x;
  if (t < cnt) {
    const int64_t g = g0 + t;
    const TileRect r = aabb_tile_rect(means2d[g * 2], means2d[g * 2 + 1], radii[g * 2], radii[g * 2 + 1], ts, tw, th);
    const int32_t off = offsets[g];
    s_off[t] = off;
    s_minx[t] = r.min_x;
    s_miny[t] = r.min_y;
    s_w[t] = r.max_x - r.min_x;
    s_hi[t] = static_cast<int64_t>(g / n_per_image) << (32 + tile_bits);
    s_bits[t] = __float_as_uint(depths[g]);
    if (t == cnt - 1) s_end = static_cast<int64_t>(off) + (r.max_y - r.min_y) * (r.max_x - r.min_x);
  }
  __syncthreads();
  // Offsets from the scan are consistent; clamping only keeps writes in
  // bounds for inconsistent caller-supplied offsets.
  const int64_t start = max<int64_t>(s_off[0], 0);
  const int64_t end = min<int64_t>(s_end, n_isects);
  for (int64_t o = start + t; o < end; o += kEncodeBlock) {
    // last j with s_off[j] <= o
    int lo = 0, hi = cnt - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_off[mid] <= o)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int j = lo;
    const int k = static_cast<int>(o - s_off[j]);
    const int w = max(s_w[j], 1);
    const int row = k / w;
    const int col = k - row * w;
    const int64_t tile = static_cast<int64_t>(s_miny[j] + row) * tw + (s_minx[j] + col);
    isect_ids[o] = s_hi[j] | (tile << 32) | static_cast<int64_t>(s_bits[j]);
    flatten_ids[o] = static_cast<int32_t>(g0 + j);
  }
}

// ---------------------------------------------------------------------------
// Depth-presorted pipeline: the sorted output of encode + stable sort by the
// 64-bit key, without sorting 64-bit keys over all intersections.
//  1. (image, gaussian) pairs are stably sorted by their depth bits (32-bit
//     keys over the I*N pairs);
//  2. the per-pair tile counts are gathered in that order and scanned;
//  3. the encoder writes each pair's tiles in depth order with 32-bit keys
//     image << tile_bits | tile;
//  4. a stable sort of those keys (image_bits + tile_bits bits, usually two
//     8-bit passes) groups entries by (image, tile) and keeps depth order
//     inside each group;
//  5. the 64-bit keys are rebuilt as key32 << 32 | depth bits.
// Equal 64-bit keys come out in ascending pair index, exactly as a stable sort
// of the encode order (pair-major) leaves them.

__global__ void __launch_bounds__(256) depth_keys_kernel(const float* __restrict__ depths, int64_t n,
                                                         uint32_t* __restrict__ keys, int32_t* __restrict__ idx) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  keys[i] = __float_as_uint(depths[i]);
  idx[i] = static_cast<int32_t>(i);
}

// Encode in depth order, balanced over ranks and outputs alike ("merge
// path"): the ranks' output starts (offsets, non-decreasing) and the output
// slots 0..n_isects-1 form one merged sequence of numel + n_isects items, rank
// r placed before slot j when offsets[r] <= j. Block b takes items
// [b K, (b+1) K): at most K slots and K ranks (plus the rank already open at
// its first slot), whatever the per-Gaussian counts, so one Gaussian with
// thousands of tiles no longer holds one block for the whole launch.

constexpr int kMergeItems = 1024;  // merged items per block
constexpr int kMergeOuts = kMergeItems / kEncodeBlock;  // slots per thread (at most)

// First r in [0, R] with offs[r] + r >= d (offs[R] + R taken as M + R), found
// by one wave in 64-way steps; every lane returns it.
__device__ int64_t merge_split(const int32_t* __restrict__ offs, int64_t R, int64_t M, int64_t d, int lane) {
  int64_t lo = max<int64_t>(0, d - M), hi = min<int64_t>(d, R);
  while (hi > lo) {
    const int64_t step = (hi - lo + kWave - 1) / kWave;
    const int64_t p = min<int64_t>(lo + lane * step, hi);
    const int64_t f = p == R ? M + R : static_cast<int64_t>(offs[p]) + p;
    const uint64_t b = __ballot(f >= d);
    if (b == 0) {
      lo = lo + (kWave - 1) * step + 1;  // after the last probe
    } else {
      const int first = __builtin_ctzll(b);
      const int64_t p_first = min<int64_t>(lo + first * step, hi);
      if (first > 0) lo = lo + (first - 1) * step + 1;
      hi = p_first;
    }
  }
  return min<int64_t>(lo, R);  // bounded even for offsets that are not a scan
}

// splits[b] = merge_split(offs, R, M, min(b * items, R + M)) for b in
// [0, nb]: every encode block's rank range found up front by one thread each
// (a binary search), so the encode blocks start without the search's chain of
// dependent loads.
__global__ void __launch_bounds__(256) merge_splits_kernel(const int32_t* __restrict__ offs, int64_t R, int64_t M,
                                                           int items, int64_t nb, int64_t* __restrict__ splits) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (b > nb) return;
  const int64_t d = min<int64_t>(b * items, R + M);
  // first r in [0, R] with offs[r] + r >= d (offs[R] + R taken as M + R)
  int64_t lo = max<int64_t>(0, d - M), hi = min<int64_t>(d, R);
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    const int64_t f = mid == R ? M + R : static_cast<int64_t>(offs[mid]) + mid;
    if (f >= d)
      hi = mid;
    else
      lo = mid + 1;
  }
  splits[b] = lo;
}

__global__ void __launch_bounds__(kEncodeBlock) encode_presorted_kernel(
    const float* __restrict__ means2d, const int32_t* __restrict__ radii, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int64_t numel, int64_t n_per_image, int ts, int tw, int th, int tile_bits,
    int64_t n_isects, uint32_t* __restrict__ keys, int32_t* __restrict__ vals, const float* __restrict__ depths,
    uint32_t* __restrict__ dbits, const int64_t* __restrict__ splits) {
  constexpr int kRanks = kMergeItems + 1;
  __shared__ int32_t s_off[kRanks];
  __shared__ uint32_t s_d[kRanks];  // depth bits (dbits set)
  __shared__ int32_t s_minx[kRanks];
  __shared__ int32_t s_miny[kRanks];
  __shared__ int32_t s_w[kRanks];
  __shared__ uint32_t s_hi[kRanks];  // image << tile_bits
  __shared__ int32_t s_g[kRanks];
  __shared__ int64_t s_split[2];
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int64_t total = numel + n_isects;
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kMergeItems;
  const int64_t d1 = min<int64_t>(d0 + kMergeItems, total);
  if (splits) {
    if (t < 2) s_split[t] = splits[blockIdx.x + t];
  } else if (wave < 2) {
    const int64_t r = merge_split(offsets, numel, n_isects, wave == 0 ? d0 : d1, lane);
    if (lane == 0) s_split[wave] = r;
  }
  __syncthreads();
  const int64_t r0 = s_split[0], r1 = s_split[1];
  const int64_t j0 = d0 - r0, j1 = d1 - r1;
  // ranks [rs, r1): the rank open at slot j0 (r0 - 1) and the ones starting in the block
  const int64_t rs = r0 > 0 ? r0 - 1 : 0;
  const int nr = static_cast<int>(min<int64_t>(max<int64_t>(r1 - rs, 0), kRanks));
  for (int i = t; i < nr; i += kEncodeBlock) {
    const int64_t g = perm[rs + i];
    TileRect rect = {0, 0, 0, 0};
    if (g >= 0 && g < numel)
      rect = aabb_tile_rect(means2d[g * 2], means2d[g * 2 + 1], radii[g * 2], radii[g * 2 + 1], ts, tw, th);
    s_off[i] = offsets[rs + i];
    s_minx[i] = rect.min_x;
    s_miny[i] = rect.min_y;
    s_w[i] = max(rect.max_x - rect.min_x, 1);
    s_hi[i] = static_cast<uint32_t>(max<int64_t>(g, 0) / n_per_image) << tile_bits;
    s_g[i] = static_cast<int32_t>(g);
    if (dbits) s_d[i] = g >= 0 && g < numel ? __float_as_uint(depths[g]) : 0u;
  }
  __syncthreads();
  if (nr == 0) return;
  // thread t owns slots j0 + t * kMergeOuts .. + kMergeOuts - 1: one binary
  // search for the first, then walk forward
  const int64_t jb = j0 + static_cast<int64_t>(t) * kMergeOuts;
  if (jb >= min<int64_t>(j1, n_isects)) return;
  int lo = 0, hi = nr - 1;  // last i with s_off[i] <= jb
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_off[mid] <= jb)
      lo = mid;
    else
      hi = mid - 1;
  }
  int i = lo;
#pragma unroll
  for (int q = 0; q < kMergeOuts; ++q) {
    const int64_t j = jb + q;
    if (j >= j1 || j >= n_isects) break;
    while (i + 1 < nr && s_off[i + 1] <= j) ++i;
    const int k = static_cast<int>(j - s_off[i]);
    const int w = s_w[i];
    const int row = k / w;
    const int col = k - row * w;
    keys[j] = s_hi[i] | static_cast<uint32_t>((s_miny[i] + row) * tw + (s_minx[i] + col));
    vals[j] = s_g[i];
    if (dbits) dbits[j] = s_d[i];
  }
}

// floor(log2(n)) + 1 with the reference's float log2 (gsplat_intersect.cpp:60-65).
int floor_log2_plus_one(int64_t value) {
  return static_cast<int>(std::floor(std::log2(static_cast<float>(value)))) + 1;
}

inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// Steps 1-2 (depth order of the pairs and the scanned counts in that order):
// workspace [dkeys | didx | dkeys_sorted | sort | scan] over numel pairs.
struct DepthOrderLayout {
  uint32_t* dkeys;
  int32_t* didx;
  uint32_t* dkeys_sorted;
  void* sort_ws;
  size_t sort_ws_bytes;
  void* scan_ws;
};

size_t depth_order_layout(int64_t numel, DepthOrderLayout* l, void* base) {
  const size_t pn = align256(static_cast<size_t>(numel) * 4);
  const size_t sort_b = align256(radix_sort_workspace_bytes<uint32_t>(numel));
  const size_t scan_b = align256(scan_workspace_bytes(numel));
  if (l && base) {
    char* p = static_cast<char*>(base);
    l->dkeys = reinterpret_cast<uint32_t*>(p);
    l->didx = reinterpret_cast<int32_t*>(p + pn);
    l->dkeys_sorted = reinterpret_cast<uint32_t*>(p + 2 * pn);
    l->sort_ws = p + 3 * pn;
    l->sort_ws_bytes = sort_b;
    l->scan_ws = p + 3 * pn + sort_b;
  }
  return 3 * pn + sort_b + scan_b;
}

// Steps 3-5 (encode in depth order, sort by (image, tile), rebuild keys):
// workspace [tkeys | tvals | tkeys_sorted | tbits | tbits_alt | sort] over
// n_isects entries. tbits carries each entry's depth bits through the sort
// passes, so the last pass writes the 64-bit ids without gathering depths.
struct EncodeSortedLayout {
  uint32_t* tkeys;
  int32_t* tvals;
  uint32_t* tkeys_sorted;
  uint32_t* tbits;
  uint32_t* tbits_alt;
  void* sort_ws;
  size_t sort_ws_bytes;
};

size_t encode_sorted_layout(int64_t n_isects, EncodeSortedLayout* l, void* base) {
  const size_t pm = align256(static_cast<size_t>(n_isects) * 4);
  const size_t sort_b = align256(radix_sort_workspace_bytes<uint32_t>(n_isects));
  if (l && base) {
    char* p = static_cast<char*>(base);
    l->tkeys = reinterpret_cast<uint32_t*>(p);
    l->tvals = reinterpret_cast<int32_t*>(p + pm);
    l->tkeys_sorted = reinterpret_cast<uint32_t*>(p + 2 * pm);
    l->tbits = reinterpret_cast<uint32_t*>(p + 3 * pm);
    l->tbits_alt = reinterpret_cast<uint32_t*>(p + 4 * pm);
    l->sort_ws = p + 5 * pm;
    l->sort_ws_bytes = sort_b;
  }
  return 5 * pm + sort_b;
}

// The encode blocks' rank ranges (merge_splits_kernel), placed in the sort
// workspace, which is free until the sort starts. NULL (the encode kernels
// then search for themselves, a few dependent loads per block) for fewer
// than kSplitMinBlocks blocks, where the extra launch costs more than the
// blocks' searches, or when they do not fit there.
constexpr int64_t kSplitMinBlocks = 65536;
// Test hook (gsplat_hip_isect_debug_set): the two size thresholds, process-wide.
std::atomic<int64_t> g_split_min_blocks{kSplitMinBlocks};

int64_t* encode_splits(const EncodeSortedLayout& l, const int32_t* offsets, int64_t numel, int64_t n_isects,
                       int items, hipStream_t s) {
  const int64_t nb = (numel + n_isects + items - 1) / items;
  if (nb < g_split_min_blocks.load(std::memory_order_relaxed) ||
      static_cast<size_t>(nb + 1) * sizeof(int64_t) > l.sort_ws_bytes)
    return nullptr;
  int64_t* splits = static_cast<int64_t*>(l.sort_ws);
  merge_splits_kernel<<<grid_for(nb + 1, 256), 256, 0, s>>>(offsets, numel, n_isects, items, nb, splits);
  return splits;
}

// Whether the tile-key passes carry each entry's depth bits (instead of the
// last pass gathering depths[flatten id]): the gather reads a cache line per
// entry at random over the depths array, cheap while that array stays in L2
// (sh3_1m's 4 MB), costly beyond (heavy_6m's 24 MB: 4.7 ms against 1.8 ms).
constexpr int64_t kCarryBitsMinPairs = int64_t{1} << 21;  // 8 MiB of depths
std::atomic<int64_t> g_carry_min_pairs{kCarryBitsMinPairs};

inline bool carry_depth_bits(int64_t numel) { return numel > g_carry_min_pairs.load(std::memory_order_relaxed); }

// Whether the carrying sorts generate their first pass's keys instead of
// encoding them (radix_sort_tiles_generated; test hook
// gsplat_hip_isect_debug_generated). It needs room for two 16-byte records
// per Gaussian in the encode's key and value buffers, so at least four
// entries per Gaussian.
std::atomic<int32_t> g_generated{1};

inline bool generate_keys(int64_t numel, int64_t n_isects, int tw, int th, int bit_hi) {
  return g_generated.load(std::memory_order_relaxed) != 0 && 4 * numel <= n_isects &&
         tiles_generated_supported(n_isects, tw, th, bit_hi);
}

int check_tile_bits(int64_t I, int32_t tile_width, int32_t tile_height, int* tile_bits, int* image_bits) {
  const int64_t n_tiles = static_cast<int64_t>(tile_width) * tile_height;
  *tile_bits = floor_log2_plus_one(n_tiles);
  *image_bits = floor_log2_plus_one(I);
  if (*image_bits + *tile_bits > 32)
    return invalid("intersect_tile_encode image id and tile id require more than 32 bits.");
  return GSPLAT_OK;
}

// Encode of the ellipse tiles, balanced like encode_presorted_kernel (merge
// path over ranks and output slots). Rank r is pair perm[r], or pair r when
// perm is NULL (the unsorted encode order). With keys32 the output is the
// 32-bit key image << tile_bits | tile for the (image, tile) sort; else ids64
// gets the full 64-bit id with the depth bits. Each thread locates its first
// slot's tile by walking the Gaussian's rows and steps along the row for the
// next ones.
constexpr int kEllItems = 512;                     // merged items per block
constexpr int kEllOuts = kEllItems / kEncodeBlock;  // slots per thread (at most)

__global__ void __launch_bounds__(kEncodeBlock) encode_ellipse_kernel(
    const float* __restrict__ means2d, const int32_t* __restrict__ radii, const float* __restrict__ conics,
    const float* __restrict__ opacities, const float* __restrict__ depths, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ image_ids, int64_t numel, int64_t n_per_image,
    int ts, int tw, int th, int tile_bits, int64_t n_isects, uint32_t* __restrict__ keys32,
    int64_t* __restrict__ ids64, int32_t* __restrict__ vals, uint32_t* __restrict__ dbits,
    const int64_t* __restrict__ splits) {
  constexpr int kRanks = kEllItems + 1;
  __shared__ int32_t s_off[kRanks];
  __shared__ int32_t s_g[kRanks];
  __shared__ EllipseTiles s_e[kRanks];  // each rank's geometry, computed once
  __shared__ int64_t s_split[2];
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int64_t total = numel + n_isects;
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kEllItems;
  const int64_t d1 = min<int64_t>(d0 + kEllItems, total);
  if (splits) {
    if (t < 2) s_split[t] = splits[blockIdx.x + t];
  } else if (wave < 2) {
    const int64_t r = merge_split(offsets, numel, n_isects, wave == 0 ? d0 : d1, lane);
    if (lane == 0) s_split[wave] = r;
  }
  __syncthreads();
  const int64_t r0 = s_split[0], r1 = s_split[1];
  const int64_t j0 = d0 - r0, j1 = d1 - r1;
  const int64_t rs = r0 > 0 ? r0 - 1 : 0;
  const int nr = static_cast<int>(min<int64_t>(max<int64_t>(r1 - rs, 0), kRanks));
  for (int i = t; i < nr; i += kEncodeBlock) {
    const int32_t g = perm ? perm[rs + i] : static_cast<int32_t>(rs + i);
    s_off[i] = offsets[rs + i];
    s_g[i] = g;
    EllipseTiles e = {};
    if (g >= 0 && g < numel) e = ellipse_tiles(means2d, radii, conics, opacities, g, ts, tw, th);
    s_e[i] = e;
  }
  __syncthreads();
  if (nr == 0) return;
  const int64_t jb = j0 + static_cast<int64_t>(t) * kEllOuts;
  if (jb >= min<int64_t>(j1, n_isects)) return;
  int lo = 0, hi = nr - 1;  // last i with s_off[i] <= jb
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_off[mid] <= jb)
      lo = mid;
    else
      hi = mid - 1;
  }
  int i = lo, cur = -1;
  EllipseTiles e = {};
  bool valid = false, ok = false;
  int ty = 0, tx = 0, row_end = 0;
  for (int q = 0; q < kEllOuts; ++q) {
    const int64_t j = jb + q;
    if (j >= j1 || j >= n_isects) break;
    while (i + 1 < nr && s_off[i + 1] <= j) ++i;
    const int64_t g = s_g[i];
    if (i != cur) {
      cur = i;
      valid = g >= 0 && g < numel;
      ok = false;
      if (valid) {
        e = s_e[i];
        ok = ellipse_locate(e, ts, static_cast<int>(j - s_off[i]), &ty, &tx, &row_end);
      }
    } else if (ok && ++tx >= row_end) {
      ok = false;
      for (int y = ty + 1; y < e.r.max_y && !ok; ++y) {
        int c0, c1;
        ellipse_row(e, y, ts, &c0, &c1);
        if (c1 > c0) {
          ty = y;
          tx = c0;
          row_end = c1;
          ok = true;
        }
      }
    }
    // offsets that disagree with the counts still get an in-range tile
    const int tile = valid && ok ? ty * tw + tx : 0;
    const uint32_t image =
        !valid ? 0u : static_cast<uint32_t>(image_ids ? static_cast<int64_t>(image_ids[g]) : g / n_per_image);
    const uint32_t key = (image << tile_bits) | static_cast<uint32_t>(tile);
    if (keys32) {
      keys32[j] = key;
      if (dbits) dbits[j] = valid ? __float_as_uint(depths[g]) : 0u;
    } else {
      const uint32_t bits = valid ? __float_as_uint(depths[g]) : 0u;
      ids64[j] = static_cast<int64_t>((static_cast<uint64_t>(key) << 32) | bits);
    }
    vals[j] = static_cast<int32_t>(g);
  }
}

// Tile offsets as lower_bound over the sorted ids (gsplat_intersect.cpp:605-641):
// one lane per offset slot o binary-searches ids >> 32 for its search key
// (o / n_tiles) << tile_bits | (o % n_tiles). The slots are few (images x
// tiles) against the ids, so the searches' reads (log2 n each, the top levels
// shared through the cache) cost far less than a pass over all ids.
__global__ void __launch_bounds__(256) offsets_search_kernel(const int64_t* __restrict__ ids, int64_t n,
                                                             int tile_bits, int64_t n_tiles, int64_t n_offsets,
                                                             int32_t* __restrict__ out) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= n_offsets) return;
  const int64_t key = ((o / n_tiles) << tile_bits) | (o % n_tiles);
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if ((ids[mid] >> 32) < key)
      lo = mid + 1;
    else
      hi = mid;
  }
  out[o] = static_cast<int32_t>(lo);
}

__global__ void fill_i32_kernel(int32_t* __restrict__ out, int64_t n, int32_t value) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = value;
}

}  // namespace
}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" size_t gsplat_hip_isect_count_scan_workspace_size(int64_t numel) { return scan_workspace_bytes(numel); }

template <bool ELL>
static int count_scan_impl(const float* means2d, const int32_t* radii, const float* conics, const float* opacities,
                           int64_t numel, int32_t tile_size, int32_t tile_width, int32_t tile_height,
                           int32_t* tiles_per_gauss, int32_t* offsets, int64_t* total_dev, void* workspace,
                           size_t workspace_bytes, void* stream) {
  hipStream_t s = as_stream(stream);
  if (numel < 0 || tile_size <= 0 || tile_width <= 0 || tile_height <= 0)
    return invalid("intersect_tile_count: invalid sizes.");
  if (!total_dev) return invalid("intersect_tile_count: null total.");
  if (numel == 0) return fill_zero(total_dev, sizeof(int64_t), s);
  if (!means2d || !radii || !tiles_per_gauss) return invalid("intersect_tile_count: null pointer.");
  if (ELL && (!conics || !opacities)) return invalid("intersect_tile_count: null conics or opacities.");
  if (!workspace || workspace_bytes < scan_workspace_bytes(numel)) {
    set_error("intersect_tile_count: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  const int64_t nb = scan_num_blocks(numel);
  int64_t* sums = static_cast<int64_t*>(workspace);
  {
    KernelTimer timer("isect_count_scan", s);
    if (ELL)
      count_scan_ellipse_kernel<<<static_cast<unsigned>(nb), kScanBlock, 0, s>>>(
          means2d, radii, conics, opacities, numel, tile_size, tile_width, tile_height, tiles_per_gauss, offsets,
          sums);
    else
      count_scan_local_kernel<<<static_cast<unsigned>(nb), kScanBlock, 0, s>>>(
          means2d, radii, numel, tile_size, tile_width, tile_height, tiles_per_gauss, offsets, sums);
  }
  int rc = check_launch("intersect_tile_count");
  if (rc) return rc;
  {
    KernelTimer timer("scan_block_sums", s);
    block_sums_scan_kernel<<<1, kScanBlock, 0, s>>>(sums, nb, total_dev);
  }
  rc = check_launch("intersect_tile_offsets (block sums)");
  if (rc || nb == 1 || !offsets) return rc;
  {
    KernelTimer timer("scan_fixup", s);
    add_block_prefix_kernel<<<static_cast<unsigned>(nb), kScanBlock, 0, s>>>(offsets, numel, sums);
  }
  return check_launch("intersect_tile_offsets (fixup)");
}

extern "C" int gsplat_hip_isect_count_scan(const float* means2d, const int32_t* radii, int64_t numel,
                                           int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                           int32_t* tiles_per_gauss, int32_t* offsets, int64_t* total_dev,
                                           void* workspace, size_t workspace_bytes, void* stream) {
  return count_scan_impl<false>(means2d, radii, nullptr, nullptr, numel, tile_size, tile_width, tile_height,
                                tiles_per_gauss, offsets, total_dev, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_isect_count_scan_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                                    const float* opacities, int64_t numel, int32_t tile_size,
                                                    int32_t tile_width, int32_t tile_height, int32_t* tiles_per_gauss,
                                                    int32_t* offsets, int64_t* total_dev, void* workspace,
                                                    size_t workspace_bytes, void* stream) {
  return count_scan_impl<true>(means2d, radii, conics, opacities, numel, tile_size, tile_width, tile_height,
                               tiles_per_gauss, offsets, total_dev, workspace, workspace_bytes, stream);
}

extern "C" int gsplat_hip_isect_encode(const float* means2d, const int32_t* radii, const float* depths,
                                       const int32_t* offsets, int64_t I, int64_t numel, int32_t tile_size,
                                       int32_t tile_width, int32_t tile_height, int64_t n_isects, int64_t* isect_ids,
                                       int32_t* flatten_ids, void* stream) {
  if (I <= 0 || numel < 0 || numel % I != 0)
    return invalid("intersect_tile_encode dense path expects depths size to equal I * N.");
  if (tile_size <= 0 || tile_width <= 0 || tile_height <= 0) return invalid("intersect_tile_encode: invalid tiles.");
  if (n_isects < 0) return invalid("intersect_tile_encode expects non-negative total_isects.");
  const int64_t n_tiles = static_cast<int64_t>(tile_width) * tile_height;
  const int tile_bits = floor_log2_plus_one(n_tiles);
  const int image_bits = floor_log2_plus_one(I);
  if (image_bits + tile_bits > 32)
    return invalid("intersect_tile_encode image id and tile id require more than 32 bits.");
  if (numel == 0 || n_isects == 0) return GSPLAT_OK;
  if (!means2d || !radii || !depths || !offsets || !isect_ids || !flatten_ids)
    return invalid("intersect_tile_encode: null pointer.");
  const int64_t nb = (numel + kEncodeG - 1) / kEncodeG;
  {
    KernelTimer timer("isect_encode", as_stream(stream));
    encode_kernel<<<static_cast<unsigned>(nb), kEncodeBlock, 0, as_stream(stream)>>>(
        means2d, radii, depths, offsets, numel, numel / I, tile_size, tile_width, tile_height, tile_bits, n_isects,
        isect_ids, flatten_ids);
  }
  return check_launch("intersect_tile_encode");
}

extern "C" int gsplat_hip_isect_offset(const int64_t* isect_ids, int64_t n_isects, int32_t I, int32_t tile_width,
                                       int32_t tile_height, int32_t* offsets, void* stream) {
  if (I <= 0 || tile_width <= 0 || tile_height <= 0)
    return invalid("intersect_offset expects positive image and tile dimensions.");
  if (n_isects < 0) return invalid("intersect_offset: negative size.");
  hipStream_t s = as_stream(stream);
  const int64_t n_tiles = static_cast<int64_t>(tile_width) * tile_height;
  const int64_t n_offsets = n_tiles * I;
  if (!offsets) return invalid("intersect_offset: null pointer.");
  if (n_isects == 0) {
    {
      KernelTimer timer("isect_offsets", s);
      fill_i32_kernel<<<grid_for(n_offsets, 256), 256, 0, s>>>(offsets, n_offsets, 0);
    }
    return check_launch("intersect_offset (empty)");
  }
  if (!isect_ids) return invalid("intersect_offset: null pointer.");
  const int tile_bits = floor_log2_plus_one(n_tiles);
  {
    KernelTimer timer("isect_offsets", s);
    offsets_search_kernel<<<grid_for(n_offsets, 256), 256, 0, s>>>(isect_ids, n_isects, tile_bits, n_tiles, n_offsets,
                                                                  offsets);
  }
  return check_launch("intersect_offset");
}

extern "C" size_t gsplat_hip_isect_depth_order_workspace_size(int64_t numel) {
  if (numel <= 0) return 0;
  return depth_order_layout(numel, nullptr, nullptr);
}

extern "C" int gsplat_hip_isect_depth_order(const float* depths, const int32_t* tiles_per_gauss, int64_t numel,
                                            int32_t* perm, int32_t* offsets, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  const char* what = "intersect_tile";
  if (numel < 0) return invalid("intersect_tile: negative size.");
  if (numel > INT32_MAX) return invalid("intersect_tile: more than 2^31-1 entries.");
  if (numel == 0) return GSPLAT_OK;
  if (!depths || !tiles_per_gauss || !perm || !offsets) return invalid("intersect_tile: null pointer.");
  DepthOrderLayout l;
  if (!workspace || workspace_bytes < depth_order_layout(numel, &l, workspace)) {
    set_error("intersect_tile: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  hipStream_t s = as_stream(stream);
  int rc;
  {
    KernelTimer timer("isect_depth_keys", s);
    depth_keys_kernel<<<grid_for(numel, 256), 256, 0, s>>>(depths, numel, l.dkeys, l.didx);
  }
  if ((rc = check_launch(what))) return rc;
  // the last pass also gathers the counts into depth order
  if ((rc = radix_sort_pairs<uint32_t>(l.dkeys, l.didx, numel, 0, 32, l.dkeys_sorted, perm, l.sort_ws,
                                       l.sort_ws_bytes, s, what, nullptr, nullptr, tiles_per_gauss, offsets)))
    return rc;
  return scan_exclusive_i32(offsets, offsets, numel, nullptr, l.scan_ws, s);
}

extern "C" size_t gsplat_hip_isect_encode_sorted_workspace_size(int64_t n_isects) {
  if (n_isects <= 0) return 0;
  return encode_sorted_layout(n_isects, nullptr, nullptr);
}

extern "C" int gsplat_hip_isect_encode_sorted(const float* means2d, const int32_t* radii, const float* depths,
                                              const int32_t* perm, const int32_t* offsets, int64_t I, int64_t numel,
                                              int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                              int64_t n_isects, int64_t* isect_ids, int32_t* flatten_ids,
                                              void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "intersect_tile";
  if (I <= 0 || numel < 0 || numel % I != 0)
    return invalid("intersect_tile dense path expects depths size to equal I * N.");
  if (tile_size <= 0 || tile_width <= 0 || tile_height <= 0) return invalid("intersect_tile: invalid tiles.");
  if (n_isects < 0) return invalid("intersect_tile: negative intersection count.");
  if (numel > INT32_MAX || n_isects > INT32_MAX) return invalid("intersect_tile: more than 2^31-1 entries.");
  int tile_bits, image_bits, rc;
  if ((rc = check_tile_bits(I, tile_width, tile_height, &tile_bits, &image_bits))) return rc;
  if (numel == 0 || n_isects == 0) return GSPLAT_OK;
  if (!means2d || !radii || !depths || !perm || !offsets || !isect_ids || !flatten_ids)
    return invalid("intersect_tile: null pointer.");
  EncodeSortedLayout l;
  if (!workspace || workspace_bytes < encode_sorted_layout(n_isects, &l, workspace)) {
    set_error("intersect_tile: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  hipStream_t s = as_stream(stream);
  const bool carry = carry_depth_bits(numel);
  if (carry && generate_keys(numel, n_isects, tile_width, tile_height, image_bits + tile_bits))
    return radix_sort_tiles_generated(means2d, radii, depths, perm, offsets, numel, numel / I, tile_size, tile_width,
                                      tile_height, tile_bits, n_isects, image_bits + tile_bits,
                                      reinterpret_cast<uint4*>(l.tkeys), reinterpret_cast<int32_t*>(l.tbits),
                                      l.tkeys_sorted, flatten_ids, isect_ids, l.tbits, l.tbits_alt, l.sort_ws,
                                      l.sort_ws_bytes, s, what);
  {
    KernelTimer timer("isect_encode", s);
    const int64_t nb = (numel + n_isects + kMergeItems - 1) / kMergeItems;
    const int64_t* splits = encode_splits(l, offsets, numel, n_isects, kMergeItems, s);
    encode_presorted_kernel<<<static_cast<unsigned>(nb), kEncodeBlock, 0, s>>>(
        means2d, radii, perm, offsets, numel, numel / I, tile_size, tile_width, tile_height, tile_bits, n_isects,
        l.tkeys, l.tvals, depths, carry ? l.tbits : nullptr, splits);
  }
  if ((rc = check_launch(what))) return rc;
  // the last pass writes the 64-bit ids (key << 32 | depth bits) directly
  return radix_sort_pairs<uint32_t>(l.tkeys, l.tvals, n_isects, 0, image_bits + tile_bits, l.tkeys_sorted,
                                    flatten_ids, l.sort_ws, l.sort_ws_bytes, s, what, depths, isect_ids, nullptr,
                                    nullptr, carry ? l.tbits : nullptr, carry ? l.tbits_alt : nullptr);
}

// Ellipse tiles, unsorted: entries in pair-major, row-major order like
// gsplat_hip_isect_encode; offsets from gsplat_hip_isect_count_scan_accutile.
extern "C" int gsplat_hip_isect_encode_accutile(const float* means2d, const int32_t* radii, const float* conics,
                                                const float* opacities, const float* depths, const int32_t* offsets,
                                                int64_t I, int64_t numel, int32_t tile_size, int32_t tile_width,
                                                int32_t tile_height, int64_t n_isects, int64_t* isect_ids,
                                                int32_t* flatten_ids, void* stream) {
  if (I <= 0 || numel < 0 || numel % I != 0)
    return invalid("intersect_tile_encode dense path expects depths size to equal I * N.");
  if (tile_size <= 0 || tile_width <= 0 || tile_height <= 0) return invalid("intersect_tile_encode: invalid tiles.");
  if (n_isects < 0) return invalid("intersect_tile_encode expects non-negative total_isects.");
  if (numel > INT32_MAX || n_isects > INT32_MAX) return invalid("intersect_tile: more than 2^31-1 entries.");
  int tile_bits, image_bits, rc;
  if ((rc = check_tile_bits(I, tile_width, tile_height, &tile_bits, &image_bits))) return rc;
  if (numel == 0 || n_isects == 0) return GSPLAT_OK;
  if (!means2d || !radii || !conics || !opacities || !depths || !offsets || !isect_ids || !flatten_ids)
    return invalid("intersect_tile_encode: null pointer.");
  hipStream_t s = as_stream(stream);
  {
    KernelTimer timer("isect_encode", s);
    const int64_t nb = (numel + n_isects + kEllItems - 1) / kEllItems;
    encode_ellipse_kernel<<<static_cast<unsigned>(nb), kEncodeBlock, 0, s>>>(
        means2d, radii, conics, opacities, depths, nullptr, offsets, nullptr, numel, numel / I, tile_size, tile_width,
        tile_height, tile_bits, n_isects, nullptr, isect_ids, flatten_ids, nullptr, nullptr);
  }
  return check_launch("intersect_tile_encode");
}

// Ellipse tiles, sorted: gsplat_hip_isect_encode_sorted with the ellipse
// tiles (perm and offsets from gsplat_hip_isect_depth_order over the counts
// of gsplat_hip_isect_count_scan_accutile).
extern "C" int gsplat_hip_isect_encode_sorted_accutile(const float* means2d, const int32_t* radii,
                                                       const float* conics, const float* opacities,
                                                       const float* depths, const int32_t* perm,
                                                       const int32_t* offsets, int64_t I, int64_t numel,
                                                       int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                                       int64_t n_isects, int64_t* isect_ids, int32_t* flatten_ids,
                                                       void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "intersect_tile";
  if (I <= 0 || numel < 0 || numel % I != 0)
    return invalid("intersect_tile dense path expects depths size to equal I * N.");
  if (tile_size <= 0 || tile_width <= 0 || tile_height <= 0) return invalid("intersect_tile: invalid tiles.");
  if (n_isects < 0) return invalid("intersect_tile: negative intersection count.");
  if (numel > INT32_MAX || n_isects > INT32_MAX) return invalid("intersect_tile: more than 2^31-1 entries.");
  int tile_bits, image_bits, rc;
  if ((rc = check_tile_bits(I, tile_width, tile_height, &tile_bits, &image_bits))) return rc;
  if (numel == 0 || n_isects == 0) return GSPLAT_OK;
  if (!means2d || !radii || !conics || !opacities || !depths || !perm || !offsets || !isect_ids || !flatten_ids)
    return invalid("intersect_tile: null pointer.");
  EncodeSortedLayout l;
  if (!workspace || workspace_bytes < encode_sorted_layout(n_isects, &l, workspace)) {
    set_error("intersect_tile: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  hipStream_t s = as_stream(stream);
  const bool carry = carry_depth_bits(numel);
  {
    KernelTimer timer("isect_encode", s);
    const int64_t nb = (numel + n_isects + kEllItems - 1) / kEllItems;
    const int64_t* splits = encode_splits(l, offsets, numel, n_isects, kEllItems, s);
    encode_ellipse_kernel<<<static_cast<unsigned>(nb), kEncodeBlock, 0, s>>>(
        means2d, radii, conics, opacities, depths, perm, offsets, nullptr, numel, numel / I, tile_size, tile_width,
        tile_height, tile_bits, n_isects, l.tkeys, nullptr, l.tvals, carry ? l.tbits : nullptr, splits);
  }
  if ((rc = check_launch(what))) return rc;
  return radix_sort_pairs<uint32_t>(l.tkeys, l.tvals, n_isects, 0, image_bits + tile_bits, l.tkeys_sorted,
                                    flatten_ids, l.sort_ws, l.sort_ws_bytes, s, what, depths, isect_ids, nullptr,
                                    nullptr, carry ? l.tbits : nullptr, carry ? l.tbits_alt : nullptr);
}

// Packed layout (IntersectTileParams.packed, gsplat_intersect.cpp:115-118):
// entry i of the nnz rows belongs to image image_ids[i]; flatten ids are
// row indices. With conics and opacities the ellipse tiles, else the AABB
// rect. Counts come from gsplat_hip_isect_count_scan(_accutile) over the
// rows, the sorted path's perm and offsets from gsplat_hip_isect_depth_order.
static int encode_packed_args(const char* what, const int32_t* image_ids, int64_t I, int64_t nnz, int32_t ts,
                              int32_t tw, int32_t th, int64_t n_isects, int* tile_bits, int* image_bits) {
  if (I <= 0 || nnz < 0) return invalid(std::string(what) + " packed path expects I > 0 and nnz >= 0.");
  if (ts <= 0 || tw <= 0 || th <= 0) return invalid(std::string(what) + ": invalid tiles.");
  if (n_isects < 0) return invalid(std::string(what) + ": negative intersection count.");
  if (nnz > INT32_MAX || n_isects > INT32_MAX) return invalid(std::string(what) + ": more than 2^31-1 entries.");
  if (nnz > 0 && n_isects > 0 && !image_ids) return invalid(std::string(what) + ": null image_ids.");
  return check_tile_bits(I, tw, th, tile_bits, image_bits);
}

extern "C" int gsplat_hip_isect_encode_packed(const float* means2d, const int32_t* radii, const float* conics,
                                              const float* opacities, const int32_t* image_ids, const float* depths,
                                              const int32_t* offsets, int64_t I, int64_t nnz, int32_t tile_size,
                                              int32_t tile_width, int32_t tile_height, int64_t n_isects,
                                              int64_t* isect_ids, int32_t* flatten_ids, void* stream) {
  int tile_bits, image_bits;
  int rc = encode_packed_args("intersect_tile_encode", image_ids, I, nnz, tile_size, tile_width, tile_height,
                              n_isects, &tile_bits, &image_bits);
  if (rc) return rc;
  if (nnz == 0 || n_isects == 0) return GSPLAT_OK;
  if (!means2d || !radii || !depths || !offsets || !isect_ids || !flatten_ids)
    return invalid("intersect_tile_encode: null pointer.");
  hipStream_t s = as_stream(stream);
  {
    KernelTimer timer("isect_encode", s);
    const int64_t nb = (nnz + n_isects + kEllItems - 1) / kEllItems;
    encode_ellipse_kernel<<<static_cast<unsigned>(nb), kEncodeBlock, 0, s>>>(
        means2d, radii, conics && opacities ? conics : nullptr, conics && opacities ? opacities : nullptr, depths,
        nullptr, offsets, image_ids, nnz, nnz, tile_size, tile_width, tile_height, tile_bits, n_isects, nullptr,
        isect_ids, flatten_ids, nullptr, nullptr);
  }
  return check_launch("intersect_tile_encode");
}

extern "C" int gsplat_hip_isect_encode_sorted_packed(const float* means2d, const int32_t* radii, const float* conics,
                                                     const float* opacities, const int32_t* image_ids,
                                                     const float* depths, const int32_t* perm, const int32_t* offsets,
                                                     int64_t I, int64_t nnz, int32_t tile_size, int32_t tile_width,
                                                     int32_t tile_height, int64_t n_isects, int64_t* isect_ids,
                                                     int32_t* flatten_ids, void* workspace, size_t workspace_bytes,
                                                     void* stream) {
  const char* what = "intersect_tile";
  int tile_bits, image_bits;
  int rc = encode_packed_args(what, image_ids, I, nnz, tile_size, tile_width, tile_height, n_isects, &tile_bits,
                              &image_bits);
  if (rc) return rc;
  if (nnz == 0 || n_isects == 0) return GSPLAT_OK;
  if (!means2d || !radii || !depths || !perm || !offsets || !isect_ids || !flatten_ids)
    return invalid("intersect_tile: null pointer.");
  EncodeSortedLayout l;
  if (!workspace || workspace_bytes < encode_sorted_layout(n_isects, &l, workspace)) {
    set_error("intersect_tile: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  hipStream_t s = as_stream(stream);
  const bool carry = carry_depth_bits(nnz);
  {
    KernelTimer timer("isect_encode", s);
    const int64_t nb = (nnz + n_isects + kEllItems - 1) / kEllItems;
    const int64_t* splits = encode_splits(l, offsets, nnz, n_isects, kEllItems, s);
    encode_ellipse_kernel<<<static_cast<unsigned>(nb), kEncodeBlock, 0, s>>>(
        means2d, radii, conics && opacities ? conics : nullptr, conics && opacities ? opacities : nullptr, depths,
        perm, offsets, image_ids, nnz, nnz, tile_size, tile_width, tile_height, tile_bits, n_isects, l.tkeys, nullptr,
        l.tvals, carry ? l.tbits : nullptr, splits);
  }
  if ((rc = check_launch(what))) return rc;
  return radix_sort_pairs<uint32_t>(l.tkeys, l.tvals, n_isects, 0, image_bits + tile_bits, l.tkeys_sorted,
                                    flatten_ids, l.sort_ws, l.sort_ws_bytes, s, what, depths, isect_ids, nullptr,
                                    nullptr, carry ? l.tbits : nullptr, carry ? l.tbits_alt : nullptr);
}

// One call: [perm | offsets | shared phase workspace] (the two phases run in
// stream order, so their scratch overlaps).
static size_t tile_sorted_layout(int64_t numel, int64_t n_isects, int32_t** perm, int32_t** offs, void** phase,
                                 void* base) {
  const size_t pn = align256(static_cast<size_t>(numel) * 4);
  if (base) {
    char* p = static_cast<char*>(base);
    *perm = reinterpret_cast<int32_t*>(p);
    *offs = reinterpret_cast<int32_t*>(p + pn);
    *phase = p + 2 * pn;
  }
  return 2 * pn + std::max(depth_order_layout(numel, nullptr, nullptr), encode_sorted_layout(n_isects, nullptr, nullptr));
}

extern "C" size_t gsplat_hip_isect_tile_sorted_workspace_size(int64_t numel, int64_t n_isects) {
  if (numel <= 0 || n_isects <= 0) return 0;
  return tile_sorted_layout(numel, n_isects, nullptr, nullptr, nullptr, nullptr);
}

extern "C" int gsplat_hip_isect_tile_sorted(const float* means2d, const int32_t* radii, const float* depths,
                                            const int32_t* tiles_per_gauss, int64_t I, int64_t numel,
                                            int32_t tile_size, int32_t tile_width, int32_t tile_height,
                                            int64_t n_isects, int64_t* isect_ids, int32_t* flatten_ids,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  if (I <= 0 || numel < 0 || numel % I != 0)
    return invalid("intersect_tile dense path expects depths size to equal I * N.");
  if (tile_size <= 0 || tile_width <= 0 || tile_height <= 0) return invalid("intersect_tile: invalid tiles.");
  if (n_isects < 0) return invalid("intersect_tile: negative intersection count.");
  if (numel > INT32_MAX || n_isects > INT32_MAX) return invalid("intersect_tile: more than 2^31-1 entries.");
  int tile_bits, image_bits, rc;
  if ((rc = check_tile_bits(I, tile_width, tile_height, &tile_bits, &image_bits))) return rc;
  if (numel == 0 || n_isects == 0) return GSPLAT_OK;
  if (!means2d || !radii || !depths || !tiles_per_gauss || !isect_ids || !flatten_ids)
    return invalid("intersect_tile: null pointer.");
  int32_t *perm = nullptr, *offs = nullptr;
  void* phase = nullptr;
  const size_t need = tile_sorted_layout(numel, n_isects, &perm, &offs, &phase, workspace);
  if (!workspace || workspace_bytes < need) {
    set_error("intersect_tile: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  const size_t phase_bytes = workspace_bytes - (static_cast<char*>(phase) - static_cast<char*>(workspace));
  if ((rc = gsplat_hip_isect_depth_order(depths, tiles_per_gauss, numel, perm, offs, phase, phase_bytes, stream)))
    return rc;
  return gsplat_hip_isect_encode_sorted(means2d, radii, depths, perm, offs, I, numel, tile_size, tile_width,
                                        tile_height, n_isects, isect_ids, flatten_ids, phase, phase_bytes, stream);
}

extern "C" void gsplat_hip_isect_debug_set(int64_t carry_min_pairs, int64_t split_min_blocks) {
  g_carry_min_pairs.store(carry_min_pairs < 0 ? kCarryBitsMinPairs : carry_min_pairs, std::memory_order_relaxed);
  g_split_min_blocks.store(split_min_blocks < 0 ? kSplitMinBlocks : split_min_blocks, std::memory_order_relaxed);
}

extern "C" void gsplat_hip_isect_debug_generated(int32_t enable) {
  g_generated.store(enable != 0 ? 1 : 0, std::memory_order_relaxed);
}

extern "C" void gsplat_hip_isect_debug_reset(void) {
  gsplat_hip_isect_debug_set(-1, -1);
  gsplat_hip_isect_debug_generated(1);
}
