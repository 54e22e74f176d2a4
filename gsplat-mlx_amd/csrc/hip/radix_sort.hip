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

template <typename K, bool ASM, bool GATHER, bool V2>
__global__ void __launch_bounds__(kSortBlock) onesweep_kernel(const K* __restrict__ keys_in,
                                                              const int32_t* __restrict__ vals_in,
                                                              const uint32_t* __restrict__ v2_in, int64_t n,
                                                              int shift, const uint32_t* __restrict__ hist,
                                                              uint32_t* __restrict__ lookback, int spin_limit,
                                                              OsOut<K> out, uint32_t dxor) {
  __shared__ K s_keys[kOsTile];
  __shared__ int32_t s_vals[kOsTile];
  __shared__ uint32_t s_v2[V2 ? kOsTile : 1];
  __shared__ uint32_t s_wcnt[kWaves][kRadix];  // per-wave running counts, then per-wave bases
  __shared__ uint32_t s_tile_start[kRadix];
  __shared__ uint32_t s_gbase[kRadix];
  __shared__ uint32_t s_wsum[kWaves];
  __shared__ uint32_t s_hsum[kWaves];
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int64_t part = blockIdx.x;
  const int64_t base = part * kOsTile;
  const int cnt = static_cast<int>(min<int64_t>(kOsTile, n - base));
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
  K k[kOsItems];
  int32_t v[kOsItems];
  uint32_t w2[V2 ? kOsItems : 1];
  uint32_t rank[kOsItems];
#pragma unroll
  for (int r = 0; r < kOsItems; ++r) {
    const int idx = wave * kOsWaveKeys + r * kWave + lane;
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
  for (int r = 0; r < kOsItems; ++r) {
    const bool valid = wave * kOsWaveKeys + r * kWave + lane < cnt;
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
  for (int r = 0; r < kOsItems; ++r) {
    if (wave * kOsWaveKeys + r * kWave + lane < cnt) {
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
    for (int64_t i = t; i < base; i += kSortBlock) atomicAdd(&wc[digit_of(kin[i], shift) ^ dxor], 1u);
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
