// A per-device cache of one device address (a `__device__` array's address on
// each GPU): filled once per device, under a mutex, by a caller-supplied lookup
// that runs with that device current.  Plain C++ (no HIP types), so the
// bookkeeping builds and is tested with g++ on a machine without a GPU.
#pragma once

#include <mutex>

namespace abacus {

template <int kSlots>
class PerDeviceAddress {
 public:
  static constexpr int kMaxDevice = kSlots - 1;

  // The cached address for device `dev`; the first call for a device runs
  // lookup(dev) -> void* and caches a non-null result.  nullptr when `dev` is
  // outside [0, kSlots) or the lookup fails (a failed lookup is retried on the
  // next call).
  template <class Lookup>
  void* get(int dev, Lookup&& lookup) {
    if (dev < 0 || dev >= kSlots) return nullptr;
    std::lock_guard<std::mutex> lock(mu_);
    if (addr_[dev] == nullptr) addr_[dev] = lookup(dev);
    return addr_[dev];
  }

 private:
  std::mutex mu_;
  void* addr_[kSlots] = {};
};

}  // namespace abacus
