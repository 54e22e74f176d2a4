// Error plumbing and small utility kernels shared by every entry point.
#include "common.hpp"

namespace gsplat_hip {

namespace {
thread_local std::string g_last_error;

__global__ void fill_zero_u32(uint32_t* __restrict__ p, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

__global__ void fill_zero_u8(uint8_t* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}
}  // namespace

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
    const int64_t n = bytes / 4;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    fill_zero_u32<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(static_cast<uint32_t*>(ptr), n);
  } else {
    fill_zero_u8<<<grid_for(bytes, 256), 256, 0, stream>>>(static_cast<uint8_t*>(ptr), bytes);
  }
  return check_launch("fill_zero");
}

}  // namespace gsplat_hip

extern "C" const char* gsplat_hip_last_error(void) { return gsplat_hip::g_last_error.c_str(); }

extern "C" int gsplat_hip_abi_version(void) { return 100; }
