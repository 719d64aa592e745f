// mk_once.h — per-device "done once" flags for host-side set-up that the HIP
// runtime keeps per device (a kernel attribute, a symbol address).  Host
// code only; no HIP calls, so it is unit-tested with a plain C++ compiler.
#pragma once
#include <atomic>
#include <cstdint>
#include <mutex>
#include <vector>

namespace mk {

class PerDeviceFlag {
 public:
  // True once set(dev) has run for this device.
  bool is_set(int dev) {
    if (dev < 0) return false;
    if (dev < 64) return (low_.load(std::memory_order_acquire) >> dev) & 1u;
    std::lock_guard<std::mutex> lock(mu_);
    return dev - 64 < (int)high_.size() && high_[dev - 64];
  }
  void set(int dev) {
    if (dev < 0) return;
    if (dev < 64) {
      low_.fetch_or(1ull << dev, std::memory_order_release);
      return;
    }
    std::lock_guard<std::mutex> lock(mu_);
    if ((int)high_.size() <= dev - 64) high_.resize(dev - 63, 0);
    high_[dev - 64] = 1;
  }

 private:
  std::atomic<uint64_t> low_{0};
  std::mutex mu_;
  std::vector<char> high_;
};

}  // namespace mk
