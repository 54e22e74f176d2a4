// Internal helpers of the C++ operator layer: device / dtype checks, stream
// selection, C-ABI status -> exception, and output allocation.
#pragma once

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <stdexcept>
#include <string>

#include "gsplat_common.h"
#include "gsplat_hip.h"

namespace gsplat_core {
namespace detail {

inline bool is_empty(const array& a) { return !a.defined() || a.numel() == 0; }

inline array empty_f32() { return at::empty({0}, at::TensorOptions().dtype(at::kFloat)); }

// The operator chain runs on ROCm devices only; there is no CPU path.
inline void require_device(const array& a, const char* name) {
  if (!a.defined() || !a.is_cuda()) {
    throw std::runtime_error(std::string("gsplat_core: ") + name +
                             " must be a tensor on a ROCm GPU device (the library has no CPU path).");
  }
}

inline void require_dtype(const array& a, at::ScalarType t, const std::string& msg) {
  if (a.scalar_type() != t) throw std::runtime_error(msg);
}

inline array contig(const array& a) { return a.is_contiguous() ? a : a.contiguous(); }

// Pointer of a possibly-empty tensor (nullptr when empty).
template <typename T>
inline const T* ptr_or_null(const array& a) {
  return is_empty(a) ? nullptr : a.data_ptr<T>();
}

inline void* stream_for(const StreamOrDevice& s, const array& ref) {
  if (s.hip_stream) return s.hip_stream;
  return c10::hip::getCurrentHIPStream(ref.device().index()).stream();
}

inline void check(int rc) {
  if (rc != GSPLAT_OK) throw std::runtime_error(gsplat_hip_last_error());
}

inline at::TensorOptions f32_like(const array& ref) { return ref.options().dtype(at::kFloat); }
inline at::TensorOptions i32_like(const array& ref) { return ref.options().dtype(at::kInt); }
inline at::TensorOptions i64_like(const array& ref) { return ref.options().dtype(at::kLong); }
inline at::TensorOptions u8_like(const array& ref) { return ref.options().dtype(at::kByte); }

// bool / uint8 mask -> contiguous uint8 view
inline array mask_u8(const array& m) {
  array c = contig(m);
  if (c.scalar_type() == at::kBool) return c.view(at::kByte);
  if (c.scalar_type() == at::kByte) return c;
  return c.to(at::kByte);
}

inline std::vector<int64_t> shape_of(const array& a) { return a.sizes().vec(); }

}  // namespace detail
}  // namespace gsplat_core
