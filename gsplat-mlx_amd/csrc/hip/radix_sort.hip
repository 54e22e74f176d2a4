// Stable LSD radix sort of 32- or 64-bit keys carrying 32-bit values, for
// gfx950.
//
// The standalone entry point replaces mx::argsort + mx::take
// (gsplat_core/gsplat_intersect.cpp:266-286) with a stable sort: equal keys
// keep their input (encode) order, which for the intersection keys is
// ascending flatten_id.
//
// Only the requested key bits are sorted, 8 bits per pass. Each pass is
// reduce-then-scan with no inter-block waiting:
//   1. histogram: each block counts the digits of its kTile keys -> block_hist
//      stored digit-major ([digit][block]);
//   2. exclusive scan of block_hist -> global start of (digit, block);
//   3. scatter: each block re-reads its tile, ranks keys stably within the
//      tile (wave ballots per 8-bit digit + per-wave digit counts in LDS),
//      reorders the tile by digit in LDS, then writes each digit run to its
//      global start, so stores of one run are contiguous.
// The final pass always lands in keys_out/vals_out; inputs are not modified.
#include "radix_sort.hpp"
#include "scan.hpp"

namespace gsplat_hip {
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
                                                          int64_t num_blocks, int32_t* __restrict__ block_hist) {
  __shared__ int32_t h[kRadix];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
#pragma unroll 4
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kSortBlock + threadIdx.x;
    if (i < n) atomicAdd(&h[digit_of(keys[i], shift)], 1);
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
                                                             int32_t* __restrict__ vals_out) {
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
    const uint32_t d = digit_of(k[r], shift);
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
      const int pos = s_tile_start[digit_of(k[r], shift)] + rank[r];
      s_keys[pos] = k[r];
      s_vals[pos] = v[r];
    }
  }
  __syncthreads();
  for (int j = t; j < cnt; j += kSortBlock) {
    const K key = s_keys[j];
    const uint32_t d = digit_of(key, shift);
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

template <typename K>
struct SortWorkspace {
  K* keys_alt;
  int32_t* vals_alt;
  int32_t* hist;
  void* scan_ws;
};

inline size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

template <typename K>
size_t layout(int64_t n, SortWorkspace<K>* ws, void* base) {
  const int64_t nb = (n + kTile - 1) / kTile;
  const size_t keys_b = align_up(static_cast<size_t>(n) * sizeof(K));
  const size_t vals_b = align_up(static_cast<size_t>(n) * sizeof(int32_t));
  const size_t hist_b = align_up(static_cast<size_t>(nb) * kRadix * sizeof(int32_t));
  const size_t scan_b = align_up(scan_workspace_bytes(nb * kRadix));
  if (ws && base) {
    char* p = static_cast<char*>(base);
    ws->keys_alt = reinterpret_cast<K*>(p);
    ws->vals_alt = reinterpret_cast<int32_t*>(p + keys_b);
    ws->hist = reinterpret_cast<int32_t*>(p + keys_b + vals_b);
    ws->scan_ws = p + keys_b + vals_b + hist_b;
  }
  return keys_b + vals_b + hist_b + scan_b;
}

}  // namespace

template <typename K>
size_t radix_sort_workspace_bytes(int64_t n) {
  return n <= 0 ? 0 : layout<K>(n, nullptr, nullptr);
}

template <typename K>
int radix_sort_pairs(const K* keys_in, const int32_t* vals_in, int64_t n, int bit_lo, int bit_hi, K* keys_out,
                     int32_t* vals_out, void* workspace, size_t workspace_bytes, hipStream_t s, const char* what) {
  const std::string w(what);
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
    return check_launch(what);
  }
  SortWorkspace<K> ws;
  if (!workspace || workspace_bytes < layout<K>(n, &ws, workspace)) {
    set_error(w + ": workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
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
      hist_kernel<K><<<static_cast<unsigned>(nb), kSortBlock, 0, s>>>(src_k, n, shift, nb, ws.hist);
    }
    int rc = check_launch(what);
    if (rc) return rc;
    rc = scan_exclusive_i32(ws.hist, ws.hist, nb * kRadix, nullptr, ws.scan_ws, s);
    if (rc) return rc;
    {
      KernelTimer timer("sort_scatter", s);
      scatter_kernel<K><<<static_cast<unsigned>(nb), kSortBlock, 0, s>>>(src_k, src_v, n, shift, nb, ws.hist, dst_k,
                                                                         dst_v);
    }
    rc = check_launch(what);
    if (rc) return rc;
    src_k = dst_k;
    src_v = dst_v;
  }
  return GSPLAT_OK;
}

template size_t radix_sort_workspace_bytes<uint32_t>(int64_t);
template size_t radix_sort_workspace_bytes<uint64_t>(int64_t);
template int radix_sort_pairs<uint32_t>(const uint32_t*, const int32_t*, int64_t, int, int, uint32_t*, int32_t*,
                                        void*, size_t, hipStream_t, const char*);
template int radix_sort_pairs<uint64_t>(const uint64_t*, const int32_t*, int64_t, int, int, uint64_t*, int32_t*,
                                        void*, size_t, hipStream_t, const char*);

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
