// Stable LSD radix sort of 32- or 64-bit keys carrying 32-bit values, for
// gfx950.
//
// The standalone entry point replaces mx::argsort + mx::take
// (gsplat_core/gsplat_intersect.cpp:266-286) with a stable sort: equal keys
// keep their input (encode) order, which for the intersection keys is
// ascending flatten_id.
//
// Only the requested key bits are sorted, 8 bits per pass.
//
// Main path (fewer than 2^30 keys), one kernel per pass after one histogram
// kernel ("onesweep"):
//   0. one read of the keys builds the global digit histogram of every pass
//      (per-block rows, then a small add kernel);
//   1. per pass, block b sorts partition b of 4096 keys (workgroups are
//      dispatched in index order on each XCD, so a waiting block's
//      predecessors on its own XCD are resident or done, and no block of a
//      higher index can hold the slot a lower one needs), ranks its keys stably (each wave ranks a contiguous quarter with
//      ballots and wave-private running digit counts), publishes its digit
//      counts, and obtains the exclusive prefix over earlier partitions by
//      decoupled look-back: per digit, walk back over predecessors' published
//      words (flag | count in one 32-bit word) until one carries an inclusive
//      prefix. Every partition publishes its counts before it looks back, so
//      the walk always ends; it is additionally bounded: a digit whose
//      predecessor stays unpublished past the spin limit recounts its prefix
//      exactly from the pass input instead (waiting on nobody), so the output
//      is the same either way. The tile is then reordered by digit in LDS and
//      written out in coalesced runs.
//
// Fallback (2^30 keys or more, where a count no longer fits beside the
// flags) is reduce-then-scan with no inter-block waiting:
//   1. histogram: each block counts the digits of its kTile keys -> block_hist
//      stored digit-major ([digit][block]);
//   2. exclusive scan of block_hist -> global start of (digit, block);
//   3. scatter: each block re-reads its tile, ranks keys stably within the
//      tile (wave ballots per 8-bit digit + per-wave digit counts in LDS),
//      reorders the tile by digit in LDS, then writes each digit run to its
//      global start, so stores of one run are contiguous.
// The final pass always lands in keys_out/vals_out; inputs are not modified.
#include <algorithm>
#include <atomic>

#include "radix_sort.hpp"
#include "scan.hpp"
#include "tiles.hpp"

namespace gsplat_hip {

// Onesweep partitions that recounted a look-back prefix (per device, since
// the library was loaded); read by gsplat_hip_sort_lookback_recounts().
__device__ unsigned long long g_lookback_recounts = 0;

namespace {

constexpr int kSortBlock = 256;
constexpr int kSortItems = 16;
constexpr int kTile = kSortBlock * kSortItems;  // keys per block
constexpr int kRadix = 256;
constexpr int kWaves = kSortBlock / kWave;

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K key, int shift) {
  return static_cast<uint32_t>(key >> shift) & (kRadix - 1);
}

template <typename K>
__global__ void __launch_bounds__(kSortBlock) hist_kernel(const K* __restrict__ keys, int64_t n, int shift,
                                                          int64_t num_blocks, int32_t* __restrict__ block_hist,
                                                          uint32_t dxor) {
  __shared__ int32_t h[kRadix];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
#pragma unroll 4
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kSortBlock + threadIdx.x;
    if (i < n) atomicAdd(&h[digit_of(keys[i], shift) ^ dxor], 1);
  }
  __syncthreads();
  block_hist[static_cast<int64_t>(threadIdx.x) * num_blocks + blockIdx.x] = h[threadIdx.x];
}

template <typename K>
__global__ void __launch_bounds__(kSortBlock) scatter_kernel(const K* __restrict__ keys_in,
                                                             const int32_t* __restrict__ vals_in, int64_t n, int shift,
                                                             int64_t num_blocks,
                                                             const int32_t* __restrict__ digit_block_start,
                                                             K* __restrict__ keys_out,
                                                             int32_t* __restrict__ vals_out, uint32_t dxor) {
  __shared__ K s_keys[kTile];
  __shared__ int32_t s_vals[kTile];
  // per-wave digit counts -> per-wave digit bases; double-buffered by round
  // parity so clearing round r+1's buffer cannot race round r's readers
  __shared__ int32_t s_wcnt[2][kWaves][kRadix];
  __shared__ int32_t s_run[kRadix];           // running per-digit count over rounds
  __shared__ int32_t s_tile_start[kRadix];    // tile-local start of each digit run
  __shared__ int32_t s_global[kRadix];        // global start of (digit, block)
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  const int cnt = static_cast<int>(min<int64_t>(kTile, n - base));

  K k[kSortItems];
  int32_t v[kSortItems];
  int32_t rank[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int p = r * kSortBlock + t;
    if (p < cnt) {
      k[r] = keys_in[base + p];
      v[r] = vals_in[base + p];
    } else {
      k[r] = 0;
      v[r] = 0;
    }
  }
  s_run[t] = 0;
  s_global[t] = digit_block_start[static_cast<int64_t>(t) * num_blocks + blockIdx.x];
  const uint64_t lanes_below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));

#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    int32_t(*wc)[kRadix] = s_wcnt[r & 1];
    // clear per-wave digit counts for this round
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wc[w][t] = 0;
    __syncthreads();
    const bool valid = r * kSortBlock + t < cnt;
    const uint32_t d = digit_of(k[r], shift) ^ dxor;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    int my_rank = 0;
    if (valid) {
      my_rank = __popcll(peers & lanes_below);
      if (my_rank == 0) wc[wave][d] = __popcll(peers);
    }
    __syncthreads();
    {  // thread t owns digit t: exclusive prefix over waves, carried over rounds
      int run = s_run[t];
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int c = wc[w][t];
        wc[w][t] = run;
        run += c;
      }
      s_run[t] = run;
    }
    __syncthreads();
    rank[r] = valid ? wc[wave][d] + my_rank : 0;
  }
  // tile-local exclusive scan of digit totals (thread t = digit t)
  {
    const int c = s_run[t];
    const int inc = wave_inclusive_scan(c);
    __shared__ int32_t s_wsum[kWaves];
    if (lane == kWave - 1) s_wsum[wave] = inc;
    __syncthreads();
    int wb = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      if (w < wave) wb += s_wsum[w];
    s_tile_start[t] = wb + inc - c;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    if (r * kSortBlock + t < cnt) {
      const int pos = s_tile_start[digit_of(k[r], shift) ^ dxor] + rank[r];
      s_keys[pos] = k[r];
      s_vals[pos] = v[r];
    }
  }
  __syncthreads();
  for (int j = t; j < cnt; j += kSortBlock) {
    const K key = s_keys[j];
    const uint32_t d = digit_of(key, shift) ^ dxor;
    const int64_t dst = static_cast<int64_t>(s_global[d]) + (j - s_tile_start[d]);
    keys_out[dst] = key;
    vals_out[dst] = s_vals[j];
  }
}

template <typename K>
__global__ void copy_kernel(const K* __restrict__ k_in, const int32_t* __restrict__ v_in, int64_t n,
                            K* __restrict__ k_out, int32_t* __restrict__ v_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) {
    k_out[i] = k_in[i];
    v_out[i] = v_in[i];
  }
}

// copy_kernel when *flag is set (a device-planned sort with no pass to run:
// every key is equal, so the stable order is the input order); a grid-stride
// loop, as the grid is sized before the flag is known.
template <typename K>
__global__ void copy_if_kernel(const K* __restrict__ k_in, const int32_t* __restrict__ v_in, int64_t n,
                               K* __restrict__ k_out, int32_t* __restrict__ v_out, const uint32_t* __restrict__ flag) {
  if (*flag == 0u) return;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    k_out[i] = k_in[i];
    v_out[i] = v_in[i];
  }
}

// ---------------------------------------------------------------------------
// Onesweep pass kernels.
constexpr int kOsItems = 16;
constexpr int kOsWaveKeys = kWave * kOsItems;     // keys ranked by one wave
constexpr int kOsTile = kSortBlock * kOsItems;    // keys per partition (4096)
constexpr uint32_t kFlagAggregate = 1u << 30;     // count of this partition only
constexpr uint32_t kFlagPrefix = 2u << 30;        // inclusive prefix through this partition
constexpr uint32_t kCountMask = (1u << 30) - 1u;
constexpr int kMaxPasses = 8;
constexpr int kSpinLimit = 1 << 18;  // empty look-back polls (each followed by s_sleep 1) before a recount
constexpr int kLookbackWindow = 8;

// Global digit histograms of every pass in two steps without same-address
// atomic pile-ups: each of up to kHistBlocks blocks histograms its share of
// partitions in LDS (16 keys per lane in flight) and stores its own row of
// partial counts; then small blocks each add up kHistRowsPerAdd rows and add
// the sums into the [passes][256] totals.
constexpr int kHistBlocks = 2048;
constexpr int kHistRowsPerAdd = 32;

template <typename K>
__global__ void __launch_bounds__(kSortBlock) hist_partial_kernel(const K* __restrict__ keys, int64_t n,
                                                                  int bit_lo, int passes, int flip_pass,
                                                                  uint32_t* __restrict__ partial,
                                                                  uint32_t* __restrict__ clear, int64_t clear_words) {
  __shared__ uint32_t h[kMaxPasses][kRadix];
  const int t = threadIdx.x;
  // the totals the add kernel accumulates into, the error word and the
  // passes' look-back words start at zero (cleared here instead of a launch
  // of its own; the kernels that use them run after this one)
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kSortBlock + t; i < clear_words;
       i += static_cast<int64_t>(gridDim.x) * kSortBlock)
    clear[i] = 0u;
  for (int p = 0; p < passes; ++p) h[p][t] = 0;
  __syncthreads();
  const int64_t n_parts = (n + kOsTile - 1) / kOsTile;
  for (int64_t part = blockIdx.x; part < n_parts; part += gridDim.x) {
    const int64_t base = part * kOsTile;
    K k[kOsItems];
#pragma unroll
    for (int r = 0; r < kOsItems; ++r) {
      const int64_t i = base + r * kSortBlock + t;
      k[r] = i < n ? keys[i] : K(0);
    }
#pragma unroll
    for (int r = 0; r < kOsItems; ++r) {
      if (base + r * kSortBlock + t >= n) continue;
      for (int p = 0; p < passes; ++p)
        atomicAdd(&h[p][digit_of(k[r], bit_lo + 8 * p) ^ (p == flip_pass ? 0x80u : 0u)], 1u);
    }
  }
  __syncthreads();
  for (int p = 0; p < passes; ++p) partial[(static_cast<int64_t>(blockIdx.x) * kMaxPasses + p) * kRadix + t] = h[p][t];
}

__global__ void __launch_bounds__(kSortBlock) hist_add_kernel(const uint32_t* __restrict__ partial, int rows,
                                                              uint32_t* __restrict__ hist) {
  const int p = blockIdx.y;
  const int t = threadIdx.x;
  const int r0 = blockIdx.x * kHistRowsPerAdd;
  const int r1 = min(rows, r0 + kHistRowsPerAdd);
  uint32_t sum = 0;
  for (int r = r0; r < r1; ++r) sum += partial[(static_cast<int64_t>(r) * kMaxPasses + p) * kRadix + t];
  if (sum) atomicAdd(&hist[p * kRadix + t], sum);
}

// Pass plan of a sort whose constant digits are found on the device (one
// thread): a digit is constant when the pass histogram counts all n keys in
// the digit of the first key; such a pass would be the identity and is
// skipped. plan[p] = 1 for a skipped pass, else src << 1 | dst << 3 with
// buffers 0 = the input, 1 = the workspace copy, 2 = the output, chosen so
// that the last pass run writes the output; plan[passes] = 1 when no pass
// runs (the output is then a copy of the input).
template <typename K>
__global__ void sort_plan_kernel(const K* __restrict__ keys, int64_t n, int bit_lo, int passes, int flip_pass,
                                 const uint32_t* __restrict__ hist, uint32_t* __restrict__ plan) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const K k0 = keys[0];
  uint32_t skip = 0;
  int runs = 0;
  for (int p = 0; p < passes; ++p) {
    const uint32_t d = digit_of(k0, bit_lo + 8 * p) ^ (p == flip_pass ? 0x80u : 0u);
    if (static_cast<int64_t>(hist[p * kRadix + d]) == n) {
      skip |= 1u << p;
    } else {
      ++runs;
    }
  }
  uint32_t src = 0;
  int j = 0;
  for (int p = 0; p < passes; ++p) {
    if ((skip >> p) & 1u) {
      plan[p] = 1u;
      continue;
    }
    const uint32_t dst = ((runs - 1 - j) % 2 == 0) ? 2u : 1u;
    plan[p] = (src << 1) | (dst << 3);
    src = dst;
    ++j;
  }
  plan[passes] = runs == 0 ? 1u : 0u;
}

// Where a pass writes: keys and values; or (ASM, 32-bit keys, last pass of
// the intersection sort) 64-bit ids key << 32 | depth bits of the value's
// pair plus the values; GATHER adds gather[value] at the same position. With
// V2 a second 32-bit value rides along (v2 in, out.v2 out); ASM then takes
// the depth bits from it instead of gathering depths[value].
// Generated first pass (radix_sort_tiles_generated): the keys of the
// depth-presorted tile lists are formed inside the first onesweep pass
// instead of being written by an encode kernel and read back. Partition p
// holds entries [4096 p, 4096 p + 4096) of the lists in depth order; entry j
// belongs to the last depth rank r with offsets[r] <= j, whose Gaussian
// g = perm[r] covers the tiles of its rect row by row: local index
// k = j - offsets[r] is tile (min_y + k / w, min_x + k % w). The entry's key
// is image << tile_bits | tile id, its value g and its carried bits the
// depth bits of g.
struct TileGenArgs {
  const int32_t* offsets;    // [numel] first entry of each rank
  const uint4* ranked;       // [numel] per rank: min_x | min_y << 16, width | height << 16 (the rect of its
                             // Gaussian in tile units), depth bits, Gaussian
  const int32_t* part_rank;  // [n_parts + 1] rank holding each partition's first entry, then numel - 1
  int64_t numel;
  int64_t n_per_image;
  int32_t tw, tile_bits;
};

// Ranks staged in LDS per chunk of a generated partition of `items` keys
// per thread (six words each: first entry, Gaussian, min corner, width,
// depth bits, image bits, in the space the partition's reorder uses
// afterwards).
constexpr int gen_ranks(int items) { return (3 * kSortBlock * items - 1) / 6; }
// Keys per thread of a generated pass: 3072 per partition, whose 42 KB of
// LDS let three blocks share a CU (two at 4096); measured faster at
// heavy_6m's sizes (2.60 against 2.90 ms) although its runs per digit are
// shorter.
constexpr int kGenItems = 12;
constexpr int kGenTile = kSortBlock * kGenItems;

// Adds the low-digit counts of the contiguous keys [a, a + len) to a
// difference array over the 256 digits (diff[d] - diff[d - 1] adds to digit
// d) plus a count added to every digit (all).
__device__ __forceinline__ void add_low_digits(uint32_t* diff, uint32_t& all, uint32_t a, uint32_t len) {
  all += len >> 8;
  const uint32_t rem = len & 255u;
  if (rem == 0u) return;
  const uint32_t s = a & 255u, e = s + rem;
  atomicAdd(&diff[s], 1u);
  if (e < 256u) {
    atomicAdd(&diff[e], ~0u);
  } else if (e > 256u) {
    atomicAdd(&diff[0], 1u);
    atomicAdd(&diff[e - 256u], ~0u);
  }
}

// floor(k / w), k - w floor(k / w) for 0 <= k, 1 <= w: the float quotient is
// within one of the exact one while k < 2^24, then corrected.
__device__ __forceinline__ void div_rect(int32_t k, int32_t w, int32_t* q, int32_t* r) {
  if (k < (1 << 24)) {
    int32_t qq = static_cast<int32_t>(floorf(static_cast<float>(k) * __builtin_amdgcn_rcpf(static_cast<float>(w))));
    int32_t rr = k - qq * w;
    if (rr < 0) {
      --qq;
      rr += w;
    } else if (rr >= w) {
      ++qq;
      rr -= w;
    }
    *q = qq;
    *r = rr;
  } else {
    *q = k / w;
    *r = k - *q * w;
  }
}

template <typename K>
struct OsOut {
  K* keys;
  int32_t* vals;
  const float* depths;    // ASM without V2: ids = key << 32 | bits of depths[value]
  int64_t* ids;
  const int32_t* gather;  // GATHER: gathered = gather[value] beside the keys
  int32_t* gathered;
  uint32_t* v2;           // V2, not ASM: the second value's output
  // device-planned passes (sort_plan_kernel; plain passes only): this pass's
  // plan entry picks the source among the input, keys_alt / vals_alt and
  // keys / vals, and the destination among the last two, or skips the pass
  const uint32_t* plan;
  K* keys_alt;
  int32_t* vals_alt;
};

// GEN: the partition's keys, values and carried bits are generated from
// `gen` (TileGenArgs; 32-bit keys with carried bits, first pass only)
// instead of read from keys_in / vals_in / v2_in.
template <typename K, bool ASM, bool GATHER, bool V2, bool GEN = false, int ITEMS = kOsItems>
__global__ void __launch_bounds__(kSortBlock) onesweep_kernel(const K* __restrict__ keys_in,
                                                              const int32_t* __restrict__ vals_in,
                                                              const uint32_t* __restrict__ v2_in, int64_t n,
                                                              int shift, const uint32_t* __restrict__ hist,
                                                              uint32_t* __restrict__ lookback, int spin_limit,
                                                              OsOut<K> out, uint32_t dxor, TileGenArgs gen = {}) {
  static_assert(!GEN || (sizeof(K) == 4 && V2 && !GATHER), "generated passes carry bits beside 32-bit keys");
  constexpr int kTileT = kSortBlock * ITEMS;  // keys per partition
  constexpr int kWaveKeysT = kWave * ITEMS;   // keys ranked by one wave
  constexpr int kPoolWords = (static_cast<int>(sizeof(K)) / 4 + 1 + (V2 ? 1 : 0)) * kTileT;
  constexpr int kGenRanksT = gen_ranks(ITEMS);
  static_assert(!GEN || kPoolWords >= 6 * kGenRanksT + 1, "generated ranks fit the reorder space");
  __shared__ __align__(16) uint32_t s_pool[kPoolWords];  // the reorder: keys, values, carried bits
  K* s_keys = reinterpret_cast<K*>(s_pool);
  int32_t* s_vals = reinterpret_cast<int32_t*>(s_pool + kTileT * sizeof(K) / 4);
  uint32_t* s_v2 = s_pool + kTileT * (sizeof(K) / 4 + 1);
  __shared__ uint32_t s_wcnt[kWaves][kRadix];  // per-wave running counts, then per-wave bases
  __shared__ uint32_t s_tile_start[kRadix];
  __shared__ uint32_t s_gbase[kRadix];
  __shared__ uint32_t s_wsum[kWaves];
  __shared__ uint32_t s_hsum[kWaves];
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int64_t part = blockIdx.x;
  const int64_t base = part * kTileT;
  const int cnt = static_cast<int>(min<int64_t>(kTileT, n - base));
  const K* kin = keys_in;
  const int32_t* vin = vals_in;
  K* kout = out.keys;
  int32_t* vout = out.vals;
  if (out.plan) {  // block-uniform
    const uint32_t e = *out.plan;
    if (e & 1u) return;  // constant digit: the pass is skipped
    const uint32_t src = (e >> 1) & 3u, dst = (e >> 3) & 3u;
    kin = src == 0u ? keys_in : (src == 1u ? out.keys_alt : out.keys);
    vin = src == 0u ? vals_in : (src == 1u ? out.vals_alt : out.vals);
    kout = dst == 1u ? out.keys_alt : out.keys;
    vout = dst == 1u ? out.vals_alt : out.vals;
  }

  // load: wave w owns tile keys [w * 1024, (w + 1) * 1024), round r covers
  // w * 1024 + r * 64 + lane, so (wave, round, lane) is input order
  K k[ITEMS];
  int32_t v[ITEMS];
  uint32_t w2[V2 ? ITEMS : 1];
  uint32_t rank[ITEMS];
  if constexpr (GEN) {
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
      k[r] = 0;
      v[r] = 0;
      w2[r] = 0;
    }
    // the partition's ranks [r0, r1], staged kGenRanksT at a time
    int32_t* g_off = reinterpret_cast<int32_t*>(s_pool);  // [kGenRanksT + 1]
    int32_t* g_g = g_off + kGenRanksT + 1;
    uint32_t* g_xy = reinterpret_cast<uint32_t*>(g_g + kGenRanksT);
    int32_t* g_w = reinterpret_cast<int32_t*>(g_xy + kGenRanksT);
    uint32_t* g_d = reinterpret_cast<uint32_t*>(g_w + kGenRanksT);
    uint32_t* g_hi = g_d + kGenRanksT;
    const int64_t r0 = gen.part_rank[part], r1 = gen.part_rank[part + 1];
    for (int64_t c0 = r0; c0 <= r1; c0 += kGenRanksT) {
      const int nc = static_cast<int>(min<int64_t>(kGenRanksT, r1 + 1 - c0));
      __syncthreads();  // the previous chunk's reads are done
      for (int i = t; i < nc; i += kSortBlock) {
        const uint4 rec = gen.ranked[c0 + i];
        g_off[i] = gen.offsets[c0 + i];
        g_g[i] = static_cast<int32_t>(rec.w);
        g_xy[i] = rec.x;
        g_w[i] = static_cast<int32_t>(max(rec.y & 0xffffu, 1u));
        g_d[i] = rec.z;
        g_hi[i] = static_cast<uint32_t>(static_cast<int64_t>(rec.w) / gen.n_per_image) << gen.tile_bits;
      }
      if (t == 0) g_off[nc] = c0 + nc < gen.numel ? gen.offsets[c0 + nc] : INT32_MAX;
      __syncthreads();
      const int32_t lo = g_off[0], hi = g_off[nc];
      // each item's rank, the last staged one whose first entry is <= j, by
      // binary lifting: the same uniform steps for all items, so the sixteen
      // items' LDS reads of a step are in flight together
      int at[ITEMS];
#pragma unroll
      for (int r = 0; r < ITEMS; ++r) at[r] = 0;
      for (int step = nc > 1 ? 1 << (31 - __builtin_clz(nc - 1)) : 0; step > 0; step >>= 1) {
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) {
          const int32_t j = static_cast<int32_t>(base + wave * kWaveKeysT + r * kWave + lane);
          const int c = at[r] + step;
          if (c < nc && g_off[c] <= j) at[r] = c;
        }
      }
#pragma unroll
      for (int r = 0; r < ITEMS; ++r) {
        const int idx = wave * kWaveKeysT + r * kWave + lane;
        const int32_t j = static_cast<int32_t>(base + idx);
        if (idx < cnt && j >= lo && j < hi) {
          const int a = at[r];
          int32_t row, col;
          div_rect(j - g_off[a], g_w[a], &row, &col);
          const uint32_t xy = g_xy[a];
          k[r] = g_hi[a] | static_cast<uint32_t>((static_cast<int32_t>(xy >> 16) + row) * gen.tw +
                                                 static_cast<int32_t>(xy & 0xffffu) + col);
          v[r] = g_g[a];
          w2[r] = g_d[a];
        }
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
      const int idx = wave * kWaveKeysT + r * kWave + lane;
      if (idx < cnt) {
        k[r] = kin[base + idx];
        v[r] = vin[base + idx];
        if constexpr (V2) w2[r] = v2_in[base + idx];
      } else {
        k[r] = 0;
        v[r] = 0;
        if constexpr (V2) w2[r] = 0;
      }
    }
  }
  // thread t owns digit t: start of digit t over the whole pass (scan of the
  // pass histogram), kept in a register until the look-back adds the prefix
  const uint32_t hc = hist[t];
  const int hinc = wave_inclusive_scan(static_cast<int>(hc));
  if (lane == kWave - 1) s_hsum[wave] = static_cast<uint32_t>(hinc);
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s_wcnt[w][t] = 0;
  __syncthreads();
  uint32_t gstart = static_cast<uint32_t>(hinc) - hc;
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w < wave) gstart += s_hsum[w];

  const uint64_t lanes_below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  uint32_t* wc = s_wcnt[wave];
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    const bool valid = wave * kWaveKeysT + r * kWave + lane < cnt;
    const uint32_t d = digit_of(k[r], shift) ^ dxor;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    // all lanes read the wave's running count of their digit, then one lane
    // per digit advances it; a wave's LDS accesses complete in issue order
    const uint32_t my = static_cast<uint32_t>(__popcll(peers & lanes_below));
    const uint32_t cur = valid ? wc[d] : 0u;
    rank[r] = cur + my;
    if (valid && my == 0) wc[d] = cur + static_cast<uint32_t>(__popcll(peers));
  }
  __syncthreads();
  // per-wave exclusive bases of digit t and the partition's count of it
  uint32_t total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const uint32_t c = s_wcnt[w][t];
    s_wcnt[w][t] = total;
    total += c;
  }
  // publish this partition's count as early as possible
  uint32_t* my_word = lookback + part * kRadix + t;
  __hip_atomic_store(my_word, (part == 0 ? kFlagPrefix : kFlagAggregate) | total, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  {
    // partition-local exclusive start of digit t (scan of the counts)
    const int inc = wave_inclusive_scan(static_cast<int>(total));
    if (lane == kWave - 1) s_wsum[wave] = static_cast<uint32_t>(inc);
    __syncthreads();
    uint32_t wb = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      if (w < wave) wb += s_wsum[w];
    s_tile_start[t] = wb + static_cast<uint32_t>(inc) - total;
  }
  __syncthreads();
  // reorder the partition by digit in LDS before looking back, so the keys
  // leave registers while earlier partitions publish
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    if (wave * kWaveKeysT + r * kWave + lane < cnt) {
      const uint32_t d = digit_of(k[r], shift) ^ dxor;
      const uint32_t pos = s_tile_start[d] + wc[d] + rank[r];
      s_keys[pos] = k[r];
      s_vals[pos] = v[r];
      if constexpr (V2) s_v2[pos] = w2[r];
    }
  }
  uint32_t prefix = 0;
  bool gave_up = part > 0 && spin_limit < 0;  // negative limit: always recount (test hook)
  if (part > 0 && !gave_up) {
    // read kLookbackWindow predecessors per step (loads in flight together);
    // positions before partition 0 read as an empty prefix
    int64_t p = part - 1;
    int spins = 0;
    for (;;) {
      uint32_t x[kLookbackWindow];
#pragma unroll
      for (int i = 0; i < kLookbackWindow; ++i)
        x[i] = p - i >= 0 ? __hip_atomic_load(lookback + (p - i) * kRadix + t, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : kFlagPrefix;
      int used = 0;
      bool done = false;
#pragma unroll
      for (int i = 0; i < kLookbackWindow; ++i) {
        if (done || used < i) continue;  // stop at the first prefix or the first word not yet published
        const uint32_t flag = x[i] & ~kCountMask;
        if (flag == 0) continue;
        prefix += x[i] & kCountMask;
        used = i + 1;
        if (flag == kFlagPrefix) done = true;
      }
      if (done) break;
      p -= used;
      if (used == 0) {
        if (++spins > spin_limit) {
          gave_up = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    if (!gave_up)
      __hip_atomic_store(my_word, kFlagPrefix | (prefix + total), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  s_gbase[t] = gstart + prefix;
  if (__syncthreads_or(gave_up)) {
    // A digit's look-back met a predecessor that had not published within
    // the spin limit (a stalled or descheduled workgroup). Its exclusive
    // prefix is then recounted exactly from the pass input, which no kernel
    // writes during the pass: the block histograms keys [0, base) into
    // per-wave LDS rows (the ranking counts are dead once the partition sits
    // reordered in LDS), and each digit that gave up takes that count. This
    // waits on no other workgroup, so the pass always ends with the same
    // output as the look-back would have given.
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s_wcnt[w][t] = 0;
    __syncthreads();
    if constexpr (GEN) {
      // the low key digits of entries [0, base) from the ranks' rects: every
      // rank before the partition's first whole, that one up to base, row by
      // row (consecutive keys) into a difference array in row 1 and a count
      // for every digit in row 2
      uint32_t* diff = s_wcnt[1];
      uint32_t all = 0;
      const int64_t r0 = gen.part_rank[part];
      for (int64_t r = t; r <= r0; r += kSortBlock) {
        const uint4 rec = gen.ranked[r];
        const uint32_t hi_bits = static_cast<uint32_t>(static_cast<int64_t>(rec.w) / gen.n_per_image) << gen.tile_bits;
        const int32_t w = static_cast<int32_t>(rec.y & 0xffffu), h = static_cast<int32_t>(rec.y >> 16);
        const int64_t e = min<int64_t>(static_cast<int64_t>(w) * h, base - gen.offsets[r]);
        if (e <= 0) continue;
        const int32_t full = static_cast<int32_t>(e / w), rem = static_cast<int32_t>(e - static_cast<int64_t>(full) * w);
        const int32_t x0 = static_cast<int32_t>(rec.x & 0xffffu), y0 = static_cast<int32_t>(rec.x >> 16);
        for (int32_t y = 0; y <= full; ++y) {
          const int32_t len = y < full ? w : rem;
          if (len > 0)
            add_low_digits(diff, all, hi_bits | static_cast<uint32_t>((y0 + y) * gen.tw + x0),
                           static_cast<uint32_t>(len));
        }
      }
      atomicAdd(&s_wcnt[2][0], all);
      __syncthreads();
      const uint32_t all_tot = s_wcnt[2][0];
      const int inc = wave_inclusive_scan(static_cast<int>(diff[t]));
      if (lane == kWave - 1) s_wsum[wave] = static_cast<uint32_t>(inc);
      __syncthreads();
      uint32_t wb = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w)
        if (w < wave) wb += s_wsum[w];
      s_wcnt[0][t] = all_tot + wb + static_cast<uint32_t>(inc);
      s_wcnt[1][t] = 0;
      s_wcnt[2][t] = 0;
    } else {
      for (int64_t i = t; i < base; i += kSortBlock) atomicAdd(&wc[digit_of(kin[i], shift) ^ dxor], 1u);
    }
    __syncthreads();
    if (gave_up) {
      prefix = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) prefix += s_wcnt[w][t];
      __hip_atomic_store(my_word, kFlagPrefix | (prefix + total), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_gbase[t] = gstart + prefix;
    }
    if (t == 0) atomicAdd(&g_lookback_recounts, 1ull);
    __syncthreads();
  }
  for (int j = t; j < cnt; j += kSortBlock) {
    const K key = s_keys[j];
    const uint32_t d = digit_of(key, shift) ^ dxor;
    const int64_t dst = static_cast<int64_t>(s_gbase[d]) + (j - static_cast<int64_t>(s_tile_start[d]));
    // generated keys whose digits disagree with the histogram (offsets not
    // from these rects) land out of place but never out of bounds
    if constexpr (GEN) {
      if (dst < 0 || dst >= n) continue;
    }
    const int32_t val = s_vals[j];
    if constexpr (ASM && V2) {
      out.ids[dst] = static_cast<int64_t>((static_cast<uint64_t>(key) << 32) | s_v2[j]);
    } else if constexpr (ASM) {
      out.ids[dst] = static_cast<int64_t>((static_cast<uint64_t>(key) << 32) | __float_as_uint(out.depths[val]));
    } else {
      kout[dst] = key;
      if constexpr (V2) out.v2[dst] = s_v2[j];
    }
    if constexpr (GATHER) out.gathered[dst] = out.gather[val];
    vout[dst] = val;
  }
}

// Records and digit histograms of the generated tile lists, one pass over
// the Gaussians in their own order: recs[g] = (min_x | min_y << 16,
// width | height << 16, depth bits, image << tile_bits) of g's AABB tile
// rect (aabb_tile_rect, the rect the counts were taken from), and per block
// one row of partial counts per pass (as hist_partial_kernel) of g's keys:
// each rect row is a run of consecutive keys, added to the low digit through
// a difference array and to the higher digits run by run. Also clears the
// totals and look-back words, as hist_partial_kernel does.
__global__ void __launch_bounds__(kSortBlock) tile_records_kernel(
    const float* __restrict__ means2d, const int32_t* __restrict__ radii, const float* __restrict__ depths,
    int64_t numel, int64_t n_per_image, int ts, int tw, int th, int tile_bits, int passes, uint4* __restrict__ recs,
    uint32_t* __restrict__ partial, uint32_t* __restrict__ clear, int64_t clear_words) {
  __shared__ uint32_t h[kMaxPasses][kRadix];  // pass 0: the difference array
  __shared__ uint32_t s_all;
  __shared__ uint32_t s_wsum[kWaves];
  const int t = threadIdx.x;
  const int lane = t % kWave, wave = t / kWave;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kSortBlock + t; i < clear_words;
       i += static_cast<int64_t>(gridDim.x) * kSortBlock)
    clear[i] = 0u;
  for (int p = 0; p < passes; ++p) h[p][t] = 0;
  if (t == 0) s_all = 0;
  __syncthreads();
  uint32_t all = 0;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kSortBlock + t; g < numel;
       g += static_cast<int64_t>(gridDim.x) * kSortBlock) {
    const TileRect r = aabb_tile_rect(means2d[g * 2], means2d[g * 2 + 1], radii[g * 2], radii[g * 2 + 1], ts, tw, th);
    const int w = max(r.max_x - r.min_x, 0), hh = max(r.max_y - r.min_y, 0);
    const uint32_t hi = static_cast<uint32_t>(g / n_per_image) << tile_bits;
    recs[g] = make_uint4(static_cast<uint32_t>(r.min_x) | (static_cast<uint32_t>(r.min_y) << 16),
                         static_cast<uint32_t>(w) | (static_cast<uint32_t>(hh) << 16), __float_as_uint(depths[g]), hi);
    if (w == 0) continue;
    for (int y = 0; y < hh; ++y) {
      const uint32_t a = hi | static_cast<uint32_t>((r.min_y + y) * tw + r.min_x);
      add_low_digits(h[0], all, a, static_cast<uint32_t>(w));
      for (int p = 1; p < passes; ++p) {
        const int sh = 8 * p;
        const uint64_t end = static_cast<uint64_t>(a) + static_cast<uint64_t>(w);
        for (uint64_t v = a >> sh; v <= (end - 1) >> sh; ++v) {
          const uint64_t lo = max<uint64_t>(a, v << sh), up = min<uint64_t>(end, (v + 1) << sh);
          atomicAdd(&h[p][v & (kRadix - 1)], static_cast<uint32_t>(up - lo));
        }
      }
    }
  }
  atomicAdd(&s_all, all);
  __syncthreads();
  const int inc = wave_inclusive_scan(static_cast<int>(h[0][t]));
  if (lane == kWave - 1) s_wsum[wave] = static_cast<uint32_t>(inc);
  __syncthreads();
  uint32_t wb = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w < wave) wb += s_wsum[w];
  partial[static_cast<int64_t>(blockIdx.x) * kMaxPasses * kRadix + t] = s_all + wb + static_cast<uint32_t>(inc);
  for (int p = 1; p < passes; ++p) partial[(static_cast<int64_t>(blockIdx.x) * kMaxPasses + p) * kRadix + t] = h[p][t];
}

// ranked[r] = recs[perm[r]] with the Gaussian perm[r] in place of the image
// bits: the records in depth order, so that a generated partition reads
// its ranks' records coalesced.
__global__ void __launch_bounds__(256) rank_records_kernel(const int32_t* __restrict__ perm,
                                                           const uint4* __restrict__ recs, int64_t numel,
                                                           uint4* __restrict__ ranked) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= numel) return;
  const int32_t g = perm[r];
  const uint4 rec = recs[g];
  ranked[r] = make_uint4(rec.x, rec.y, rec.z, static_cast<uint32_t>(g));
}

// part_rank[p] = the last depth rank whose first entry is <= tile p (the rank
// holding partition p's first entry), for p < n_parts; part_rank[n_parts] =
// numel - 1.
__global__ void __launch_bounds__(256) partition_ranks_kernel(const int32_t* __restrict__ offsets, int64_t numel,
                                                              int64_t n_parts, int64_t tile,
                                                              int32_t* __restrict__ part_rank) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (p > n_parts) return;
  if (p == n_parts) {
    part_rank[p] = static_cast<int32_t>(numel - 1);
    return;
  }
  const int64_t x = p * tile;
  int64_t lo = 0, hi = numel - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (offsets[mid] <= x) lo = mid; else hi = mid - 1;
  }
  part_rank[p] = static_cast<int32_t>(lo);
}

template <typename K>
struct SortWorkspace {
  K* keys_alt;
  int32_t* vals_alt;
  int32_t* hist;
  void* scan_ws;
  // onesweep
  uint32_t* os_hist;      // [kMaxPasses][256]
  uint32_t* os_lookback;  // [passes][n_parts][256]
  uint32_t* os_partial;   // [kHistBlocks][kMaxPasses][256] per-block histogram rows
  uint32_t* plan;         // [kMaxPasses + 1] device pass plan (sort_plan_kernel)
};

inline size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Keys below this count take the onesweep path (counts fit beside the flags).
constexpr int64_t kOnesweepMaxKeys = static_cast<int64_t>(1) << 30;

// Test hooks (gsplat_hip_sort_debug_set): the look-back spin limit and the
// onesweep key limit, process-wide.
std::atomic<int32_t> g_spin_limit{kSpinLimit};
std::atomic<int64_t> g_onesweep_max_keys{kOnesweepMaxKeys};

template <typename K>
size_t layout(int64_t n, SortWorkspace<K>* ws, void* base) {
  const int64_t nb = (n + kTile - 1) / kTile;
  const int64_t n_parts = (n + kOsTile - 1) / kOsTile;
  const int max_passes = static_cast<int>(sizeof(K));
  const size_t keys_b = align_up(static_cast<size_t>(n) * sizeof(K));
  const size_t vals_b = align_up(static_cast<size_t>(n) * sizeof(int32_t));
  const bool onesweep = n < g_onesweep_max_keys.load(std::memory_order_relaxed);
  const size_t hist_b = onesweep ? 0 : align_up(static_cast<size_t>(nb) * kRadix * sizeof(int32_t));
  const size_t scan_b = onesweep ? 0 : align_up(scan_workspace_bytes(nb * kRadix));
  const size_t oh_b = onesweep ? align_up(kMaxPasses * kRadix * sizeof(uint32_t)) : 0;
  const size_t ol_b = onesweep ? align_up(static_cast<size_t>(max_passes) * n_parts * kRadix * sizeof(uint32_t)) : 0;
  const size_t op_b = onesweep ? align_up(static_cast<size_t>(kHistBlocks) * kMaxPasses * kRadix * sizeof(uint32_t)) : 0;
  const size_t plan_b = align_up((kMaxPasses + 1) * sizeof(uint32_t));
  if (ws && base) {
    char* p = static_cast<char*>(base);
    ws->keys_alt = reinterpret_cast<K*>(p);
    ws->vals_alt = reinterpret_cast<int32_t*>(p + keys_b);
    ws->hist = reinterpret_cast<int32_t*>(p + keys_b + vals_b);
    ws->scan_ws = p + keys_b + vals_b + hist_b;
    char* q = p + keys_b + vals_b + hist_b + scan_b;
    ws->os_hist = reinterpret_cast<uint32_t*>(q);
    ws->os_lookback = reinterpret_cast<uint32_t*>(q + oh_b);
    ws->os_partial = reinterpret_cast<uint32_t*>(q + oh_b + ol_b);
    ws->plan = reinterpret_cast<uint32_t*>(q + oh_b + ol_b + op_b);
  }
  return keys_b + vals_b + hist_b + scan_b + oh_b + ol_b + op_b + plan_b;
}

// ids[i] = keys[i] << 32 | bits of depths[vals[i]] (32-bit keys).
template <typename K>
__global__ void __launch_bounds__(256) assemble_ids_kernel(const K* __restrict__ keys,
                                                           const int32_t* __restrict__ vals,
                                                           const float* __restrict__ depths, int64_t n,
                                                           int64_t* __restrict__ ids) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  ids[i] = static_cast<int64_t>((static_cast<uint64_t>(keys[i]) << 32) | __float_as_uint(depths[vals[i]]));
}

template <typename K>
int assemble(const K* keys, const int32_t* vals, const float* depths, int64_t n, int64_t* ids, hipStream_t s,
             const char* what) {
  {
    KernelTimer timer("sort_assemble_ids", s);
    assemble_ids_kernel<K><<<grid_for(n, 256), 256, 0, s>>>(keys, vals, depths, n, ids);
  }
  return check_launch(what);
}

// out[i] = src[idx[i]].
__global__ void __launch_bounds__(256) gather_kernel(const int32_t* __restrict__ idx, const int32_t* __restrict__ src,
                                                     int64_t n, int32_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = src[idx[i]];
}

int gather(const int32_t* idx, const int32_t* src, int64_t n, int32_t* out, hipStream_t s, const char* what) {
  {
    KernelTimer timer("sort_gather", s);
    gather_kernel<<<grid_for(n, 256), 256, 0, s>>>(idx, src, n, out);
  }
  return check_launch(what);
}

}  // namespace

template <typename K>
size_t radix_sort_workspace_bytes(int64_t n) {
  return n <= 0 ? 0 : layout<K>(n, nullptr, nullptr);
}

template <typename K>
int radix_sort_pairs(const K* keys_in, const int32_t* vals_in, int64_t n, int bit_lo, int bit_hi, K* keys_out,
                     int32_t* vals_out, void* workspace, size_t workspace_bytes, hipStream_t s, const char* what,
                     const float* asm_depths, int64_t* asm_ids, const int32_t* gather_src, int32_t* gather_dst,
                     uint32_t* asm_bits, uint32_t* asm_bits_alt) {
  const std::string w(what);
  if (asm_ids && (sizeof(K) != 4 || !asm_depths)) return invalid(w + ": invalid sort arguments.");
  if ((asm_bits || asm_bits_alt) && (!asm_ids || !asm_bits || !asm_bits_alt))
    return invalid(w + ": invalid sort arguments.");
  if (gather_dst && (asm_ids || !gather_src)) return invalid(w + ": invalid sort arguments.");
  if (n < 0 || bit_lo < 0 || bit_hi > static_cast<int>(8 * sizeof(K)) || bit_lo > bit_hi)
    return invalid(w + ": invalid sort arguments.");
  if (n == 0) return GSPLAT_OK;
  if (!keys_in || !vals_in || !keys_out || !vals_out) return invalid(w + ": null pointer.");
  if (n > (static_cast<int64_t>(1) << 31) - 1) return invalid(w + ": more than 2^31-1 keys.");
  const int passes = (bit_hi - bit_lo + 7) / 8;
  if (passes == 0) {
    {
      KernelTimer timer("sort_copy", s);
      copy_kernel<K><<<grid_for(n, 256), 256, 0, s>>>(keys_in, vals_in, n, keys_out, vals_out);
    }
    if (asm_ids) return assemble(keys_out, vals_out, asm_depths, n, asm_ids, s, what);
    if (gather_dst) return gather(vals_out, gather_src, n, gather_dst, s, what);
    return check_launch(what);
  }
  SortWorkspace<K> ws;
  if (!workspace || workspace_bytes < layout<K>(n, &ws, workspace)) {
    set_error(w + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  if (n < g_onesweep_max_keys.load(std::memory_order_relaxed)) {
    const int64_t n_parts = (n + kOsTile - 1) / kOsTile;
    const int spin = g_spin_limit.load(std::memory_order_relaxed);
    // histograms and this sort's look-back words start at zero
    const int64_t clear_words = (reinterpret_cast<char*>(ws.os_lookback + passes * n_parts * kRadix) -
                                 reinterpret_cast<char*>(ws.os_hist)) / 4;
    int rc;
    {
      KernelTimer timer("sort_histogram", s);
      const int hb = static_cast<int>(std::min<int64_t>(n_parts, kHistBlocks));
      hist_partial_kernel<K><<<static_cast<unsigned>(hb), kSortBlock, 0, s>>>(
          keys_in, n, bit_lo, passes, -1, ws.os_partial, ws.os_hist, clear_words);
      const dim3 add_grid((hb + kHistRowsPerAdd - 1) / kHistRowsPerAdd, passes);
      hist_add_kernel<<<add_grid, kSortBlock, 0, s>>>(ws.os_partial, hb, ws.os_hist);
    }
    if ((rc = check_launch(what))) return rc;
    const K* src_k = keys_in;
    const int32_t* src_v = vals_in;
    const uint32_t* src_b = asm_bits;  // the carried depth bits (asm_bits set)
    for (int p = 0; p < passes; ++p) {
      const bool to_out = ((passes - 1 - p) % 2) == 0;
      K* dst_k = to_out ? keys_out : ws.keys_alt;
      int32_t* dst_v = to_out ? vals_out : ws.vals_alt;
      // bits ping-pong between the two caller buffers; the last pass reads them
      uint32_t* dst_b = p % 2 == 0 ? asm_bits_alt : asm_bits;
      {
        KernelTimer timer("sort_onesweep", s);
        const bool last = p == passes - 1;
        const OsOut<K> o{dst_k, dst_v, asm_depths, asm_ids, gather_src, gather_dst, dst_b};
        const unsigned grid = static_cast<unsigned>(n_parts);
        const uint32_t* hist_p = ws.os_hist + p * kRadix;
        uint32_t* look_p = ws.os_lookback + p * n_parts * kRadix;
        const int shift = bit_lo + 8 * p;
        bool launched = false;
        if constexpr (sizeof(K) == 4) {
          if (last && asm_ids && asm_bits) {
            onesweep_kernel<K, true, false, true><<<grid, kSortBlock, 0, s>>>(src_k, src_v, src_b, n, shift, hist_p,
                                                                              look_p, spin, o, 0u);
            launched = true;
          } else if (last && asm_ids) {
            onesweep_kernel<K, true, false, false><<<grid, kSortBlock, 0, s>>>(src_k, src_v, nullptr, n, shift,
                                                                               hist_p, look_p, spin, o, 0u);
            launched = true;
          } else if (asm_bits) {
            onesweep_kernel<K, false, false, true><<<grid, kSortBlock, 0, s>>>(src_k, src_v, src_b, n, shift, hist_p,
                                                                               look_p, spin, o, 0u);
            launched = true;
          }
        }
        if (!launched && last && gather_dst) {
          onesweep_kernel<K, false, true, false><<<grid, kSortBlock, 0, s>>>(src_k, src_v, nullptr, n, shift, hist_p,
                                                                             look_p, spin, o, 0u);
          launched = true;
        }
        if (!launched)
          onesweep_kernel<K, false, false, false><<<grid, kSortBlock, 0, s>>>(src_k, src_v, nullptr, n, shift,
                                                                              hist_p, look_p, spin, o, 0u);
      }
      if ((rc = check_launch(what))) return rc;
      src_k = dst_k;
      src_v = dst_v;
      src_b = dst_b;
    }
    return GSPLAT_OK;
  }
  const int64_t nb = (n + kTile - 1) / kTile;
  const K* src_k = keys_in;
  const int32_t* src_v = vals_in;
  for (int p = 0; p < passes; ++p) {
    // the last pass writes keys_out: alternate so that parity works out
    const bool to_out = ((passes - 1 - p) % 2) == 0;
    K* dst_k = to_out ? keys_out : ws.keys_alt;
    int32_t* dst_v = to_out ? vals_out : ws.vals_alt;
    const int shift = bit_lo + 8 * p;
    {
      KernelTimer timer("sort_histogram", s);
      hist_kernel<K><<<static_cast<unsigned>(nb), kSortBlock, 0, s>>>(src_k, n, shift, nb, ws.hist, 0u);
    }
    int rc = check_launch(what);
    if (rc) return rc;
    rc = scan_exclusive_i32(ws.hist, ws.hist, nb * kRadix, nullptr, ws.scan_ws, s);
    if (rc) return rc;
    {
      KernelTimer timer("sort_scatter", s);
      scatter_kernel<K><<<static_cast<unsigned>(nb), kSortBlock, 0, s>>>(src_k, src_v, n, shift, nb, ws.hist, dst_k,
                                                                         dst_v, 0u);
    }
    rc = check_launch(what);
    if (rc) return rc;
    src_k = dst_k;
    src_v = dst_v;
  }
  if (asm_ids) return assemble(keys_out, vals_out, asm_depths, n, asm_ids, s, what);
  if (gather_dst) return gather(vals_out, gather_src, n, gather_dst, s, what);
  return GSPLAT_OK;
}

// Stable sort of signed 64-bit keys (two's complement order: the top digit's
// sign bit is flipped when digits are formed, the keys themselves are moved
// unchanged) over all eight digits, with the passes on digits that every key
// shares found and skipped on the device (sort_plan_kernel): nothing is read
// back to the host. Inputs of 2^30 keys or more take the block-scan passes,
// all eight of them.
int radix_sort_pairs_i64_planned(const int64_t* keys_in_s, const int32_t* vals_in, int64_t n, int64_t* keys_out_s,
                                 int32_t* vals_out, void* workspace, size_t workspace_bytes, hipStream_t s,
                                 const char* what) {
  using K = uint64_t;
  const std::string w(what);
  if (n < 0) return invalid(w + ": invalid sort arguments.");
  if (n == 0) return GSPLAT_OK;
  if (!keys_in_s || !vals_in || !keys_out_s || !vals_out) return invalid(w + ": null pointer.");
  if (n > (static_cast<int64_t>(1) << 31) - 1) return invalid(w + ": more than 2^31-1 keys.");
  const K* keys_in = reinterpret_cast<const K*>(keys_in_s);
  K* keys_out = reinterpret_cast<K*>(keys_out_s);
  constexpr int passes = 8;
  constexpr int flip_pass = passes - 1;
  SortWorkspace<K> ws;
  if (!workspace || workspace_bytes < layout<K>(n, &ws, workspace)) {
    set_error(w + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  int rc;
  if (n < g_onesweep_max_keys.load(std::memory_order_relaxed)) {
    const int64_t n_parts = (n + kOsTile - 1) / kOsTile;
    const int spin = g_spin_limit.load(std::memory_order_relaxed);
    const int64_t clear_words = (reinterpret_cast<char*>(ws.os_lookback + passes * n_parts * kRadix) -
                                 reinterpret_cast<char*>(ws.os_hist)) / 4;
    {
      KernelTimer timer("sort_histogram", s);
      const int hb = static_cast<int>(std::min<int64_t>(n_parts, kHistBlocks));
      hist_partial_kernel<K><<<static_cast<unsigned>(hb), kSortBlock, 0, s>>>(
          keys_in, n, 0, passes, flip_pass, ws.os_partial, ws.os_hist, clear_words);
      const dim3 add_grid((hb + kHistRowsPerAdd - 1) / kHistRowsPerAdd, passes);
      hist_add_kernel<<<add_grid, kSortBlock, 0, s>>>(ws.os_partial, hb, ws.os_hist);
      sort_plan_kernel<K><<<1, 64, 0, s>>>(keys_in, n, 0, passes, flip_pass, ws.os_hist, ws.plan);
    }
    if ((rc = check_launch(what))) return rc;
    for (int p = 0; p < passes; ++p) {
      KernelTimer timer("sort_onesweep", s);
      OsOut<K> o{};
      o.keys = keys_out;
      o.vals = vals_out;
      o.plan = ws.plan + p;
      o.keys_alt = ws.keys_alt;
      o.vals_alt = ws.vals_alt;
      onesweep_kernel<K, false, false, false><<<static_cast<unsigned>(n_parts), kSortBlock, 0, s>>>(
          keys_in, vals_in, nullptr, n, 8 * p, ws.os_hist + p * kRadix, ws.os_lookback + p * n_parts * kRadix, spin,
          o, p == flip_pass ? 0x80u : 0u);
      if ((rc = check_launch(what))) return rc;
    }
    {
      KernelTimer timer("sort_copy", s);
      const unsigned cg = static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 2048));
      copy_if_kernel<K><<<cg, 256, 0, s>>>(keys_in, vals_in, n, keys_out, vals_out, ws.plan + passes);
    }
    return check_launch(what);
  }
  const int64_t nb = (n + kTile - 1) / kTile;
  const K* src_k = keys_in;
  const int32_t* src_v = vals_in;
  for (int p = 0; p < passes; ++p) {
    const bool to_out = ((passes - 1 - p) % 2) == 0;
    K* dst_k = to_out ? keys_out : ws.keys_alt;
    int32_t* dst_v = to_out ? vals_out : ws.vals_alt;
    const int shift = 8 * p;
    const uint32_t dxor = p == flip_pass ? 0x80u : 0u;
    {
      KernelTimer timer("sort_histogram", s);
      hist_kernel<K><<<static_cast<unsigned>(nb), kSortBlock, 0, s>>>(src_k, n, shift, nb, ws.hist, dxor);
    }
    if ((rc = check_launch(what))) return rc;
    if ((rc = scan_exclusive_i32(ws.hist, ws.hist, nb * kRadix, nullptr, ws.scan_ws, s))) return rc;
    {
      KernelTimer timer("sort_scatter", s);
      scatter_kernel<K><<<static_cast<unsigned>(nb), kSortBlock, 0, s>>>(src_k, src_v, n, shift, nb, ws.hist, dst_k,
                                                                         dst_v, dxor);
    }
    if ((rc = check_launch(what))) return rc;
    src_k = dst_k;
    src_v = dst_v;
  }
  return GSPLAT_OK;
}

// At most three passes: the generated pass's look-back words (a third more
// partitions than a pass of 4096 keys) and the others' fit the four passes'
// words of the workspace.
bool tiles_generated_supported(int64_t n, int tw, int th, int bit_hi) {
  return n > 0 && n < g_onesweep_max_keys.load(std::memory_order_relaxed) && tw > 0 && th > 0 && tw < 65536 &&
         th < 65536 && bit_hi >= 1 && bit_hi <= 24;
}

int radix_sort_tiles_generated(const float* means2d, const int32_t* radii, const float* depths, const int32_t* perm,
                               const int32_t* offsets, int64_t numel, int64_t n_per_image, int ts, int tw, int th,
                               int tile_bits, int64_t n, int bit_hi, uint4* recs, int32_t* part_rank,
                               uint32_t* keys_out, int32_t* vals_out, int64_t* ids, uint32_t* bits,
                               uint32_t* bits_alt, void* workspace, size_t workspace_bytes, hipStream_t s,
                               const char* what) {
  using K = uint32_t;
  const std::string w(what);
  if (!tiles_generated_supported(n, tw, th, bit_hi) || numel <= 0 || numel > INT32_MAX || n_per_image <= 0)
    return invalid(w + ": invalid sort arguments.");
  if (!means2d || !radii || !depths || !perm || !offsets || !recs || !part_rank || !keys_out || !vals_out || !ids ||
      !bits || !bits_alt)
    return invalid(w + ": null pointer.");
  SortWorkspace<K> ws;
  if (!workspace || workspace_bytes < layout<K>(n, &ws, workspace)) {
    set_error(w + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  const int passes = (bit_hi + 7) / 8;
  const int64_t n_parts = (n + kOsTile - 1) / kOsTile;
  const int64_t n_gen = (n + kGenTile - 1) / kGenTile;  // partitions of the generated pass
  const int spin = g_spin_limit.load(std::memory_order_relaxed);
  // look-back words: the generated pass's, then each later pass's
  auto look = [&](int p) { return ws.os_lookback + (p == 0 ? 0 : (n_gen + (p - 1) * n_parts) * kRadix); };
  const int64_t clear_words = (reinterpret_cast<char*>(look(passes)) - reinterpret_cast<char*>(ws.os_hist)) / 4;
  int rc;
  {
    KernelTimer timer("sort_histogram", s);
    const int hb = static_cast<int>(std::min<int64_t>((numel + kSortBlock - 1) / kSortBlock, kHistBlocks));
    tile_records_kernel<<<static_cast<unsigned>(hb), kSortBlock, 0, s>>>(
        means2d, radii, depths, numel, n_per_image, ts, tw, th, tile_bits, passes, recs, ws.os_partial, ws.os_hist,
        clear_words);
    const dim3 add_grid((hb + kHistRowsPerAdd - 1) / kHistRowsPerAdd, passes);
    hist_add_kernel<<<add_grid, kSortBlock, 0, s>>>(ws.os_partial, hb, ws.os_hist);
    partition_ranks_kernel<<<grid_for(n_gen + 1, 256), 256, 0, s>>>(offsets, numel, n_gen, kGenTile, part_rank);
    rank_records_kernel<<<grid_for(numel, 256), 256, 0, s>>>(perm, recs, numel, recs + numel);
  }
  if ((rc = check_launch(what))) return rc;
  const TileGenArgs gen{offsets, recs + numel, part_rank, numel, n_per_image, tw, tile_bits};
  const K* src_k = nullptr;
  const int32_t* src_v = nullptr;
  const uint32_t* src_b = nullptr;
  for (int p = 0; p < passes; ++p) {
    const bool to_out = ((passes - 1 - p) % 2) == 0;
    K* dst_k = to_out ? keys_out : ws.keys_alt;
    int32_t* dst_v = to_out ? vals_out : ws.vals_alt;
    uint32_t* dst_b = p % 2 == 0 ? bits_alt : bits;
    {
      KernelTimer timer("sort_onesweep", s);
      const bool last = p == passes - 1;
      const OsOut<K> o{dst_k, dst_v, depths, ids, nullptr, nullptr, dst_b};
      const unsigned grid = static_cast<unsigned>(p == 0 ? n_gen : n_parts);
      const uint32_t* hist_p = ws.os_hist + p * kRadix;
      uint32_t* look_p = look(p);
      const int shift = 8 * p;
      if (p == 0 && last)
        onesweep_kernel<K, true, false, true, true, kGenItems><<<grid, kSortBlock, 0, s>>>(
            nullptr, nullptr, nullptr, n, shift, hist_p, look_p, spin, o, 0u, gen);
      else if (p == 0)
        onesweep_kernel<K, false, false, true, true, kGenItems><<<grid, kSortBlock, 0, s>>>(
            nullptr, nullptr, nullptr, n, shift, hist_p, look_p, spin, o, 0u, gen);
      else if (last)
        onesweep_kernel<K, true, false, true><<<grid, kSortBlock, 0, s>>>(src_k, src_v, src_b, n, shift, hist_p,
                                                                          look_p, spin, o, 0u);
      else
        onesweep_kernel<K, false, false, true><<<grid, kSortBlock, 0, s>>>(src_k, src_v, src_b, n, shift, hist_p,
                                                                           look_p, spin, o, 0u);
    }
    if ((rc = check_launch(what))) return rc;
    src_k = dst_k;
    src_v = dst_v;
    src_b = dst_b;
  }
  return GSPLAT_OK;
}

template size_t radix_sort_workspace_bytes<uint32_t>(int64_t);
template size_t radix_sort_workspace_bytes<uint64_t>(int64_t);
template int radix_sort_pairs<uint32_t>(const uint32_t*, const int32_t*, int64_t, int, int, uint32_t*, int32_t*,
                                        void*, size_t, hipStream_t, const char*, const float*, int64_t*,
                                        const int32_t*, int32_t*, uint32_t*, uint32_t*);
template int radix_sort_pairs<uint64_t>(const uint64_t*, const int32_t*, int64_t, int, int, uint64_t*, int32_t*,
                                        void*, size_t, hipStream_t, const char*, const float*, int64_t*,
                                        const int32_t*, int32_t*, uint32_t*, uint32_t*);

}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" size_t gsplat_hip_isect_sort_workspace_size(int64_t n) { return radix_sort_workspace_bytes<uint64_t>(n); }

extern "C" int gsplat_hip_isect_sort(const int64_t* keys_in, const int32_t* vals_in, int64_t n, int32_t key_bits,
                                     int64_t* keys_out, int32_t* vals_out, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (n < 0 || key_bits < 0 || key_bits > 64) return invalid("intersect_tile_sort: invalid arguments.");
  if (n == 0) return GSPLAT_OK;
  if (!keys_out) return invalid("intersect_tile_sort: null pointer.");
  return radix_sort_pairs<uint64_t>(reinterpret_cast<const uint64_t*>(keys_in), vals_in, n, 0, key_bits,
                                    reinterpret_cast<uint64_t*>(keys_out), vals_out, workspace, workspace_bytes,
                                    as_stream(stream), "intersect_tile_sort");
}

extern "C" int gsplat_hip_isect_sort_i64(const int64_t* keys_in, const int32_t* vals_in, int64_t n,
                                         int64_t* keys_out, int32_t* vals_out, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  return radix_sort_pairs_i64_planned(keys_in, vals_in, n, keys_out, vals_out, workspace, workspace_bytes,
                                      as_stream(stream), "intersect_tile_sort");
}

extern "C" void gsplat_hip_sort_debug_set(int32_t spin_limit, int64_t onesweep_max_keys) {
  g_spin_limit.store(spin_limit, std::memory_order_relaxed);
  g_onesweep_max_keys.store(onesweep_max_keys <= 0 ? kOnesweepMaxKeys : std::min(onesweep_max_keys, kOnesweepMaxKeys),
                            std::memory_order_relaxed);
}

extern "C" void gsplat_hip_sort_debug_reset(void) { gsplat_hip_sort_debug_set(kSpinLimit, 0); }

extern "C" int gsplat_hip_sort_lookback_recounts(uint64_t* count) {
  if (!count) return invalid("sort_lookback_recounts: null pointer.");
  unsigned long long v = 0;
  const int rc = check_hip(hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_lookback_recounts), sizeof(v), 0,
                                               hipMemcpyDeviceToHost),
                           "sort_lookback_recounts");
  if (rc) return rc;
  *count = v;
  return GSPLAT_OK;
}
