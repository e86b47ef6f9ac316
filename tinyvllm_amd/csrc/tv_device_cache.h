// Host-side values computed once per device: resident work-group counts of a
// kernel (occupancy x compute units), looked up by the launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

namespace tv {

constexpr int kMaxDevices = 64;

// Work-groups of `kernel` (launched with `threads` per work-group) resident at
// once on the current device, cached per device in `slots`.  Lock-free: host
// threads that race on the first call both compute and store the same value.
// A device index past the table is answered uncached.
template <typename K>
long long resident_work_groups(std::atomic<long long> (&slots)[kMaxDevices], K kernel, int threads) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  if (dev < kMaxDevices) {
    const long long v = slots[dev].load(std::memory_order_relaxed);
    if (v != 0) return v;
  }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
  const long long v = (long long)per_cu * cus;
  if (dev < kMaxDevices) slots[dev].store(v, std::memory_order_relaxed);
  return v;
}

}  // namespace tv
