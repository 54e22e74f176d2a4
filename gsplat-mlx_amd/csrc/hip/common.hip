// Error plumbing, opt-in kernel timing and small utility kernels shared by
// every entry point.
#include <algorithm>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.hpp"

namespace gsplat_hip {
namespace {

thread_local std::string g_last_error;

__global__ void fill_zero_u8(uint8_t* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// blockIdx.y selects the span; 16-byte stores over its aligned body, plain
// stores for the unaligned head and the tail.
__global__ void __launch_bounds__(256) fill_zero_spans_kernel(ZeroSpans z) {
  float* p = z.ptr[blockIdx.y];
  const int64_t n = z.count[blockIdx.y];
  const int64_t head = std::min<int64_t>(n, ((16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15) / 4);
  const int64_t n4 = (n - head) / 4;
  const int64_t tail = n - head - 4 * n4;
  const int t = threadIdx.x;
  if (blockIdx.x == 0 && t < head) p[t] = 0.0f;
  if (blockIdx.x == 0 && t < tail) p[head + 4 * n4 + t] = 0.0f;
  float4* q = reinterpret_cast<float4*>(p + head);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + t; i < n4; i += stride)
    q[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

struct TimedLaunch {
  const char* name;
  hipEvent_t start;
  hipEvent_t stop;
};

bool g_profile = false;
std::vector<TimedLaunch> g_pending;
std::map<std::string, std::pair<int64_t, double>> g_totals;  // name -> (launches, total ms)

void drain_pending() {
  for (const TimedLaunch& t : g_pending) {
    float ms = 0.0f;
    if (hipEventSynchronize(t.stop) == hipSuccess && hipEventElapsedTime(&ms, t.start, t.stop) == hipSuccess) {
      auto& tot = g_totals[t.name];
      tot.first += 1;
      tot.second += ms;
    }
    (void)hipEventDestroy(t.start);
    (void)hipEventDestroy(t.stop);
  }
  g_pending.clear();
}

}  // namespace

KernelTimer::KernelTimer(const char* name, hipStream_t stream) : name_(name), stream_(stream) {
  if (!g_profile) return;
  if (hipEventCreate(&start_) != hipSuccess) {
    start_ = nullptr;
    return;
  }
  if (hipEventRecord(start_, stream_) != hipSuccess) {
    (void)hipEventDestroy(start_);
    start_ = nullptr;
  }
}

KernelTimer::~KernelTimer() {
  if (!start_) return;
  hipEvent_t stop = nullptr;
  if (hipEventCreate(&stop) == hipSuccess && hipEventRecord(stop, stream_) == hipSuccess) {
    g_pending.push_back({name_, start_, stop});
    if (g_pending.size() > 4096) drain_pending();
  } else {
    (void)hipEventDestroy(start_);
    if (stop) (void)hipEventDestroy(stop);
  }
}

void set_error(const std::string& msg) { g_last_error = msg; }

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return GSPLAT_OK;
  set_error(std::string(what) + ": " + hipGetErrorString(err));
  return GSPLAT_ERR_HIP;
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

int fill_zero(void* ptr, int64_t bytes, hipStream_t stream) {
  if (bytes <= 0) return GSPLAT_OK;
  if (reinterpret_cast<uintptr_t>(ptr) % 4 == 0 && bytes % 4 == 0) {
    const ZeroSpan span{static_cast<float*>(ptr), bytes / 4};
    return fill_zero_spans(&span, 1, stream);
  }
  KernelTimer timer("fill_zero", stream);
  fill_zero_u8<<<grid_for(bytes, 256), 256, 0, stream>>>(static_cast<uint8_t*>(ptr), bytes);
  return check_launch("fill_zero");
}

int fill_zero_spans(const ZeroSpan* spans, int n_spans, hipStream_t stream) {
  const ZeroSpans z = pack_zero_spans(spans, n_spans);
  if (z.n == 0) return GSPLAT_OK;
  int64_t largest = 0;
  for (int k = 0; k < z.n; ++k) largest = std::max(largest, z.count[k]);
  KernelTimer timer("fill_zero", stream);
  // about four float4 stores per thread on the largest span
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((largest / 4 + 1023) / 1024, 4096));
  fill_zero_spans_kernel<<<dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(z.n)), 256, 0, stream>>>(z);
  return check_launch("fill_zero");
}

// Attainable FP32 VALU rate: 8 independent FMA chains per lane keep every
// SIMD issuing single (not packed) FP32 instructions; the flops per launch
// are blocks * 256 lanes * 8 chains * 2 * iters.
__global__ void __launch_bounds__(256) valu_probe_kernel(float* __restrict__ out, int iters, float b, float c) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = static_cast<float>(threadIdx.x) * 1.0e-3f + static_cast<float>(i);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = __builtin_fmaf(a[i], b, c);
  }
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sum += a[i];
  out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = sum;
}

// LDS broadcast reads, the rasterizers' record access: each wave reads 16-byte
// records at wave-uniform addresses (one address per instruction, broadcast to
// all 64 lanes), four independent reads per step, each consumed by two
// three-operand integer adds (v_add3_u32) so that the LDS reads, not the VALU,
// bound the loop. 16 KiB of records per block.
__global__ void __launch_bounds__(256) lds_probe_kernel(uint32_t* __restrict__ out, int iters) {
  __shared__ uint4 rec[1024];
  for (int i = threadIdx.x; i < 1024; i += 256)
    rec[i] = make_uint4(static_cast<uint32_t>(i), static_cast<uint32_t>(3 * i), static_cast<uint32_t>(5 * i),
                        static_cast<uint32_t>(7 * i));
  __syncthreads();
  const int base = (threadIdx.x / kWave) * 64;  // per wave, uniform
  uint32_t a[4] = {0u, 1u, 2u, 3u}, b[4] = {4u, 5u, 6u, 7u};
  for (int it = 0; it < iters; ++it) {
    const int k = (base + it * 4) & 1023;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 r = rec[k + j];
      a[j] = a[j] + r.x + r.y;
      b[j] = b[j] + r.z + r.w;
    }
  }
  uint32_t sum = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) sum += a[j] ^ b[j];
  out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = sum;
}

}  // namespace gsplat_hip

extern "C" int gsplat_hip_lds_probe(uint32_t* out, int64_t blocks, int32_t iters, void* stream) {
  if (!out || blocks <= 0 || blocks > 65535 || iters <= 0 || iters % 256 != 0)
    return gsplat_hip::invalid("lds_probe: invalid arguments.");
  gsplat_hip::lds_probe_kernel<<<static_cast<unsigned>(blocks), 256, 0, gsplat_hip::as_stream(stream)>>>(out, iters);
  return gsplat_hip::check_launch("lds_probe");
}

extern "C" int gsplat_hip_valu_probe(float* out, int64_t blocks, int32_t iters, void* stream) {
  if (!out || blocks <= 0 || blocks > 65535 || iters <= 0) return gsplat_hip::invalid("valu_probe: invalid arguments.");
  gsplat_hip::valu_probe_kernel<<<static_cast<unsigned>(blocks), 256, 0, gsplat_hip::as_stream(stream)>>>(
      out, iters, 0.999f, 0.001f);
  return gsplat_hip::check_launch("valu_probe");
}

extern "C" const char* gsplat_hip_last_error(void) { return gsplat_hip::g_last_error.c_str(); }

// 1.01: ellipse tiles, packed layout, rasterize-to-indices and selective Adam
// entry points added (additive). 1.02: allocation-free rasterize backward,
// sort diagnostics and test hooks, exp and LDS probes (additive).
// 200: gsplat_hip_sh_camera_colors_fwd takes the projection's radii (an
// argument more), the packed camera colours and the packed row kernels added
extern "C" int gsplat_hip_abi_version(void) { return 200; }

extern "C" void gsplat_hip_profile_enable(int32_t enable) { gsplat_hip::g_profile = enable != 0; }

extern "C" void gsplat_hip_profile_reset(void) {
  gsplat_hip::drain_pending();
  gsplat_hip::g_totals.clear();
}

extern "C" size_t gsplat_hip_profile_report(char* buf, size_t buf_len) {
  gsplat_hip::drain_pending();
  std::string out;
  for (const auto& kv : gsplat_hip::g_totals) {
    char line[256];
    std::snprintf(line, sizeof(line), "%s\t%lld\t%.6f\n", kv.first.c_str(), static_cast<long long>(kv.second.first),
                  kv.second.second);
    out += line;
  }
  if (buf && buf_len > 0) {
    const size_t n = std::min(out.size(), buf_len - 1);
    std::memcpy(buf, out.data(), n);
    buf[n] = '\0';
  }
  return out.size();
}
