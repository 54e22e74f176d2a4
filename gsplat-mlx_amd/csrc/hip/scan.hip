// Reduce-then-scan exclusive prefix sum of int32 values (see scan.hpp).
#include "scan.hpp"

namespace gsplat_hip {
namespace {

__global__ void __launch_bounds__(kScanBlock) scan_local_kernel(const int32_t* __restrict__ in,
                                                               int32_t* __restrict__ out, int64_t n,
                                                               int64_t* __restrict__ block_sums) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + static_cast<int64_t>(threadIdx.x) * kScanItems;
  int32_t v[kScanItems];
  int64_t sum = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    v[k] = base + k < n ? in[base + k] : 0;
    sum += v[k];
  }
  int64_t total;
  int64_t run = block_exclusive_scan(sum, &total);
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    if (base + k < n) out[base + k] = static_cast<int32_t>(run);
    run += v[k];
  }
  if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// One block: exclusive scan of the block sums in place; grand total to *total.
__global__ void __launch_bounds__(kScanBlock) scan_block_sums_kernel(int64_t* __restrict__ sums, int64_t nb,
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
  if (threadIdx.x == 0 && total_dev) *total_dev = carry;
}

__global__ void __launch_bounds__(kScanBlock) scan_fixup_kernel(int32_t* __restrict__ out, int64_t n,
                                                               const int64_t* __restrict__ block_sums) {
  const int64_t add = block_sums[blockIdx.x];
  if (add == 0) return;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  for (int k = threadIdx.x; k < kScanTile; k += kScanBlock) {
    const int64_t i = base + k;
    if (i < n) out[i] = static_cast<int32_t>(out[i] + add);
  }
}

// Small inputs (up to kSingleBlock * kSingleItems values): one block of
// 1024 threads -- one launch instead of three. The values pass through LDS so
// that global loads and stores are coalesced (wave w moves 64 consecutive
// values per instruction) while each thread scans kSingleItems consecutive
// values; a thread-strided global layout would turn every store into 64
// partial-line writes from one CU.
constexpr int kSingleBlock = 1024;
constexpr int kSingleItems = 16;
constexpr int64_t kSingleMax = static_cast<int64_t>(kSingleBlock) * kSingleItems;

__global__ void __launch_bounds__(kSingleBlock) scan_single_kernel(const int32_t* __restrict__ in,
                                                                  int32_t* __restrict__ out, int64_t n,
                                                                  int64_t* __restrict__ total_dev) {
  __shared__ int32_t s_v[kSingleMax];
  __shared__ int64_t s_wave[kSingleBlock / kWave];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int cnt = static_cast<int>(n);  // n <= kSingleMax
#pragma unroll
  for (int k = 0; k < kSingleItems; ++k) {
    const int i = k * kSingleBlock + t;
    s_v[i] = i < cnt ? in[i] : 0;
  }
  __syncthreads();  // every read of in precedes every write of out (they may alias)
  int32_t v[kSingleItems];
  int64_t sum = 0;
#pragma unroll
  for (int k = 0; k < kSingleItems; ++k) {
    v[k] = s_v[t * kSingleItems + k];
    sum += v[k];
  }
  const int64_t inc = wave_inclusive_scan_i64(sum);
  if (lane == kWave - 1) s_wave[wave] = inc;
  __syncthreads();
  int64_t run = inc - sum, tot = 0;
#pragma unroll
  for (int w = 0; w < kSingleBlock / kWave; ++w) {
    const int64_t x = s_wave[w];
    run += w < wave ? x : 0;
    tot += x;
  }
#pragma unroll
  for (int k = 0; k < kSingleItems; ++k) {
    s_v[t * kSingleItems + k] = static_cast<int32_t>(run);
    run += v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kSingleItems; ++k) {
    const int i = k * kSingleBlock + t;
    if (i < cnt) out[i] = s_v[i];
  }
  if (t == 0 && total_dev) *total_dev = tot;
}

}  // namespace

int scan_exclusive_i32(const int32_t* in, int32_t* out, int64_t n, int64_t* total_dev, void* workspace,
                       hipStream_t stream) {
  if (n <= 0) {
    if (total_dev) return fill_zero(total_dev, sizeof(int64_t), stream);
    return GSPLAT_OK;
  }
  const int64_t nb = scan_num_blocks(n);
  if (nb > kMaxGridX) return invalid("scan: too many elements.");
  if (n <= kSingleMax) {
    {
      KernelTimer timer("scan_local", stream);
      scan_single_kernel<<<1, kSingleBlock, 0, stream>>>(in, out, n, total_dev);
    }
    return check_launch("scan (single block)");
  }
  int64_t* sums = static_cast<int64_t*>(workspace);
  {
    KernelTimer timer("scan_local", stream);
    scan_local_kernel<<<static_cast<unsigned>(nb), kScanBlock, 0, stream>>>(in, out, n, sums);
  }
  int rc = check_launch("scan (local)");
  if (rc) return rc;
  {
    KernelTimer timer("scan_block_sums", stream);
    scan_block_sums_kernel<<<1, kScanBlock, 0, stream>>>(sums, nb, total_dev);
  }
  rc = check_launch("scan (block sums)");
  if (rc) return rc;
  if (nb > 1) {
    {
      KernelTimer timer("scan_fixup", stream);
      scan_fixup_kernel<<<static_cast<unsigned>(nb), kScanBlock, 0, stream>>>(out, n, sums);
    }
    rc = check_launch("scan (fixup)");
  }
  return rc;
}

}  // namespace gsplat_hip

using namespace gsplat_hip;

extern "C" size_t gsplat_hip_exclusive_scan_i32_workspace_size(int64_t n) { return scan_workspace_bytes(n); }

extern "C" int gsplat_hip_exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, int64_t* total_dev,
                                             void* workspace, size_t workspace_bytes, void* stream) {
  if (n < 0) return invalid("exclusive_scan: negative size.");
  if (n > 0 && (!in || !out)) return invalid("exclusive_scan: null pointer.");
  if (n > 0 && (!workspace || workspace_bytes < scan_workspace_bytes(n))) {
    set_error("exclusive_scan: workspace too small.");
    return GSPLAT_ERR_WORKSPACE_TOO_SMALL;
  }
  return scan_exclusive_i32(in, out, n, total_dev, workspace, as_stream(stream));
}
