// Common types of the gsplat_core C++ operator API (MI355X build).
//
// The reference API (a1091150/gsplat-mlx, gsplat_core/include/*.h) passes
// mx::array values and an mx::StreamOrDevice. This library keeps the same
// structs, field names and order, with at::Tensor (ROCm device tensors) as
// the array type and StreamOrDevice naming the HIP stream to enqueue on
// (default: the caller's current torch stream on the tensors' device).
#pragma once

#include <ATen/ATen.h>

#include <cstdint>
#include <vector>

namespace gsplat_core {

using array = at::Tensor;

struct StreamOrDevice {
  // nullptr: the current HIP stream of the input tensors' device.
  void* hip_stream = nullptr;
  StreamOrDevice() = default;
  explicit StreamOrDevice(void* s) : hip_stream(s) {}
};

}  // namespace gsplat_core
