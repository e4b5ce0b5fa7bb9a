// Host-only check of PerDeviceAddress (abacus_amd/csrc/device_table.h), the
// per-device cache behind the allocation-free router weight gradient's scratch
// lookup.  Built with g++ and run by tests/test_noalloc_plan.py; prints "ok"
// and exits 0 when every check holds.
#include <atomic>
#include <cstdio>
#include <cstdint>
#include <thread>
#include <vector>

#include "device_table.h"

#define CHECK(c)                                              \
  do {                                                        \
    if (!(c)) {                                               \
      std::printf("FAILED line %d: %s\n", __LINE__, #c);       \
      return 1;                                               \
    }                                                         \
  } while (0)

static void* addr_of(int dev) { return reinterpret_cast<void*>((uintptr_t)(0x1000 + 0x100 * dev)); }

int main() {
  abacus::PerDeviceAddress<1024> table;
  static_assert(abacus::PerDeviceAddress<1024>::kMaxDevice == 1023, "slots");
  std::vector<int> calls(1024, 0);
  auto lookup = [&](int dev) -> void* {
    ++calls[dev];
    return addr_of(dev);
  };
  // Each device, including indices past 63, gets its own address from one lookup.
  for (int dev : {0, 1, 7, 63, 64, 65, 255, 1023}) {
    CHECK(table.get(dev, lookup) == addr_of(dev));
    CHECK(table.get(dev, lookup) == addr_of(dev));
    CHECK(calls[dev] == 1);
  }
  // Out of range: no lookup, nullptr.
  int outside = 0;
  auto counting = [&](int) -> void* { ++outside; return addr_of(0); };
  CHECK(table.get(-1, counting) == nullptr);
  CHECK(table.get(1024, counting) == nullptr);
  CHECK(table.get(1 << 20, counting) == nullptr);
  CHECK(outside == 0);
  // A failed lookup is not cached: the next call looks up again.
  int tries = 0;
  auto flaky = [&](int dev) -> void* { return ++tries == 1 ? nullptr : addr_of(dev); };
  CHECK(table.get(100, flaky) == nullptr);
  CHECK(table.get(100, flaky) == addr_of(100));
  CHECK(table.get(100, flaky) == addr_of(100));
  CHECK(tries == 2);
  // Many threads asking for the same devices at once: one lookup per device.
  abacus::PerDeviceAddress<1024> shared;
  std::vector<std::atomic<int>> n(16);
  for (auto& a : n) a = 0;
  std::vector<std::thread> pool;
  std::atomic<int> wrong{0};
  for (int t = 0; t < 8; ++t)
    pool.emplace_back([&, t] {
      for (int i = 0; i < 2000; ++i) {
        const int dev = (i + t) % 16;
        void* p = shared.get(dev, [&](int d) -> void* { ++n[d]; return addr_of(d); });
        if (p != addr_of(dev)) ++wrong;
      }
    });
  for (auto& th : pool) th.join();
  CHECK(wrong == 0);
  for (auto& a : n) CHECK(a == 1);
  std::printf("ok\n");
  return 0;
}
