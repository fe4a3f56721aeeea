// Host-side facts about the current HIP device, cached per device.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

namespace akas {

constexpr int kMaxDevices = 64;

// Index of the current device, or -1 when it cannot be read or is past
// kMaxDevices.
inline int current_device() {
  int dev = -1;
  return hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices ? dev : -1;
}

// Compute units of the current device (256 when they cannot be read).
inline int device_cus() {
  static std::atomic<int> cus[kMaxDevices];
  const int dev = current_device();
  if (dev < 0) return 256;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
    c = 256;
  cus[dev].store(c, std::memory_order_relaxed);
  return c;
}

}  // namespace akas
