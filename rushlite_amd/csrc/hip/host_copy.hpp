// Host threads for the pageable half of staged host <-> device copies
// (runtime.hip): a range is split into slices copied at once by the caller and
// parked worker threads.  Plain C++, so the CPU tests can run it.
#pragma once

#include <algorithm>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <system_error>
#include <thread>

namespace lmp_hip {

constexpr unsigned kCopyThreads = 8;            // the caller included
constexpr size_t kCopySlice = size_t(1) << 20;  // least bytes per thread

// copy() splits a range into slices of at least kCopySlice bytes, runs slice 0
// on the caller and the others on parked workers, and returns when all are
// done.  Calls must not overlap (the staged copies hold their staging lock).
// One process-wide pool, immortal: its workers stay parked until the process
// ends.
class HostCopyPool {
 public:
  static HostCopyPool& get() {
    static HostCopyPool* p = new HostCopyPool();
    return *p;
  }

  // Threads this pool copies with, the caller included.
  unsigned threads() const { return workers_ + 1; }

  void copy(void* dst, const void* src, size_t n) {
    if (n == 0) return;
    const size_t most = std::max<size_t>(1, n / kCopySlice);
    const size_t want = std::min<size_t>(workers_ + 1, most);
    size_t per = (n + want - 1) / want;
    per = (per + 63) & ~size_t(63);
    const int parts = int((n + per - 1) / per);
    if (parts <= 1) {
      std::memcpy(dst, src, n);
      return;
    }
    {
      std::lock_guard<std::mutex> lock(mu_);
      dst_ = static_cast<char*>(dst);
      src_ = static_cast<const char*>(src);
      n_ = n;
      per_ = per;
      parts_ = parts;
      remaining_ = parts - 1;
      ++gen_;
    }
    start_.notify_all();
    std::memcpy(dst, src, per);
    std::unique_lock<std::mutex> lock(mu_);
    done_.wait(lock, [&] { return remaining_ == 0; });
  }

 private:
  HostCopyPool() {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned want = std::min(kCopyThreads, hw) - 1;
    // Fewer workers if the system refuses a thread (copy() uses what started).
    try {
      for (unsigned i = 0; i < want; ++i) {
        std::thread([this, i] { run(int(i) + 1); }).detach();
        workers_ = i + 1;
      }
    } catch (const std::system_error&) {
    }
  }

  // Worker `part` copies slice `part` of each job that has one.
  void run(int part) {
    uint64_t seen = 0;
    std::unique_lock<std::mutex> lock(mu_);
    for (;;) {
      start_.wait(lock, [&] { return gen_ != seen; });
      seen = gen_;
      if (part >= parts_) continue;
      char* d = dst_ + size_t(part) * per_;
      const char* s = src_ + size_t(part) * per_;
      const size_t len = std::min(per_, n_ - size_t(part) * per_);
      lock.unlock();
      std::memcpy(d, s, len);
      lock.lock();
      if (--remaining_ == 0) done_.notify_one();
    }
  }

  unsigned workers_ = 0;
  std::mutex mu_;
  std::condition_variable start_, done_;
  char* dst_ = nullptr;
  const char* src_ = nullptr;
  size_t n_ = 0, per_ = 0;
  int parts_ = 0, remaining_ = 0;
  uint64_t gen_ = 0;
};

}  // namespace lmp_hip
