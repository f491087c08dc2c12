// Host-only checks of the backend's CPU-side logic: the caching arena
// (best fit, split, coalesce, segment release, unknown-address rejection),
// its growth policy on an out-of-memory device (wait, release the cached free
// segments, retry once; allocator.cu:101-125) against a synthetic device, and
// the magic-number divider, and the host thread pool of the staged copies
// (slices of random lengths and offsets copied byte for byte).  Built and run
// by tests/test_host_native.py with g++; no GPU involved.
#include <cassert>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "arena.hpp"
#include "fastdiv.hpp"
#include "host_copy.hpp"

using lmp_hip::Arena;
using lmp_hip::DeviceAlloc;
using lmp_hip::FastDiv;

#define CHECK(c)                                                  \
  do {                                                            \
    if (!(c)) {                                                   \
      std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c);     \
      return 1;                                                   \
    }                                                             \
  } while (0)

int arena_checks() {
  Arena a(256);
  CHECK(!a.add_segment(0x1001, 4096));             // misaligned
  CHECK(a.add_segment(0x100000, 1 << 20));         // 1 MiB segment
  CHECK(!a.add_segment(0x100000 + 4096, 8192));    // overlaps
  CHECK(a.add_segment(0x400000, 1 << 16));         // 64 KiB segment
  auto z = a.allocate(0);
  CHECK(z && z->addr == 0);
  auto x = a.allocate(1000);                       // best fit: the 64 KiB segment
  CHECK(x && x->addr == 0x400000 && x->size == 1024);
  auto y = a.allocate(60000);
  CHECK(y && y->addr == 0x400400);
  auto big = a.allocate(100000);                   // only fits the 1 MiB segment
  CHECK(big && big->addr == 0x100000);
  CHECK(!a.allocate(2 << 20));                     // larger than any free block
  CHECK(a.in_use_bytes() == 1024 + 60160 + 100096);
  CHECK(!a.release(0x400010));                     // not a block start
  CHECK(a.release(x->addr));
  CHECK(!a.release(x->addr));                      // double free rejected
  CHECK(a.release(y->addr));                       // coalesces back into one block
  auto segs = a.take_free_segments();              // the 64 KiB one is whole again
  CHECK(segs.size() == 1 && segs[0].addr == 0x400000 && segs[0].size == (1u << 16));
  CHECK(a.segment_count() == 1);
  CHECK(a.release(big->addr));
  CHECK(a.free_block_count() == 1 && a.block_count() == 1);
  // random alloc/free against a shadow model: no overlaps, full coalescing
  std::mt19937 rng(7);
  Arena r(256);
  CHECK(r.add_segment(0x10000000, 64u << 20));
  std::vector<Arena::Span> live;
  for (int it = 0; it < 20000; ++it) {
    if (live.empty() || rng() % 3) {
      auto s = r.allocate(1 + rng() % 200000);
      if (s) {
        for (auto& o : live) CHECK(s->addr + s->size <= o.addr || o.addr + o.size <= s->addr);
        live.push_back(*s);
      }
    } else {
      size_t i = rng() % live.size();
      CHECK(r.release(live[i].addr));
      live.erase(live.begin() + long(i));
    }
  }
  for (auto& s : live) CHECK(r.release(s.addr));
  CHECK(r.free_block_count() == 1 && r.in_use_bytes() == 0);
  return 0;
}

// A device with `capacity` bytes: hands out aligned, non-overlapping bases,
// refuses a request that would exceed its capacity, and logs every call.
struct FakeDevice {
  std::size_t capacity, held = 0;
  Arena::Addr next = 0x40000000;
  std::vector<std::pair<Arena::Addr, std::size_t>> live;
  std::vector<std::string> log;
  bool fail_sync = false;
  Arena::Addr fail_free_of = 0;  // a release of this base fails (and keeps it)
  DeviceAlloc malloc(std::size_t bytes, Arena::Addr* base) {
    log.push_back("malloc " + std::to_string(bytes));
    if (held + bytes > capacity) return DeviceAlloc::kOutOfMemory;
    *base = next;
    next += bytes;
    held += bytes;
    live.push_back({*base, bytes});
    return DeviceAlloc::kOk;
  }
  bool sync() {
    log.push_back("sync");
    return !fail_sync;
  }
  bool free(Arena::Addr base) {
    log.push_back("free " + std::to_string(base));
    if (base == fail_free_of) return false;
    for (auto it = live.begin(); it != live.end(); ++it)
      if (it->first == base) {
        held -= it->second;
        live.erase(it);
        return true;
      }
    return false;
  }
};

int growth_policy_checks() {
  constexpr std::size_t kMin = 1 << 20;  // minimum segment
  using Log = std::vector<std::string>;
  {
    // Two cached segments: one wholly free (1 MiB), one holding a live block
    // (2 MiB).  A 1.5 MiB request fits no free block, and the 3.5 MiB device
    // has no room for a 1.5 MiB segment until the free one is given back: the
    // policy must wait, hand back exactly that segment, and retry once.
    FakeDevice dev{7 << 19};
    Arena eager(256);
    Arena::Addr a = 0, b = 0;
    CHECK(dev.malloc(kMin, &a) == DeviceAlloc::kOk && eager.add_segment(a, kMin));
    CHECK(dev.malloc(2 * kMin, &b) == DeviceAlloc::kOk && eager.add_segment(b, 2 * kMin));
    auto keep = eager.allocate(3 * kMin / 2);  // lives in the 2 MiB segment
    CHECK(keep && keep->addr == b);
    dev.log.clear();
    Arena::Span span;
    std::size_t seg = 0;
    auto st = lmp_hip::grow_and_allocate(eager, eager, 1536 << 10, kMin, true, dev, &span, &seg);
    CHECK(st == DeviceAlloc::kOk && seg == std::size_t(1536) << 10);
    CHECK((dev.log == Log{"malloc 1572864", "sync", "free " + std::to_string(a), "malloc 1572864"}));
    CHECK(eager.segment_count() == 2 && span.size == std::size_t(1536) << 10);
    CHECK(eager.release(span.addr) && eager.release(keep->addr));
  }
  {
    // Still too little after the release: one retry, then out of memory,
    // and nothing is added to the arena.
    FakeDevice dev{kMin};
    Arena eager(256);
    Arena::Addr a = 0;
    CHECK(dev.malloc(kMin, &a) == DeviceAlloc::kOk && eager.add_segment(a, kMin));
    auto keep = eager.allocate(100);
    dev.log.clear();
    Arena::Span span;
    std::size_t seg = 0;
    auto st = lmp_hip::grow_and_allocate(eager, eager, 4096, kMin, true, dev, &span, &seg);
    CHECK(st == DeviceAlloc::kOutOfMemory);
    CHECK((dev.log == Log{"malloc 1048576", "sync", "malloc 1048576"}));  // no free segment to give
    CHECK(eager.segment_count() == 1 && eager.release(keep->addr));
  }
  {
    // During a graph capture (no release allowed): no wait, no release, one
    // request only; a graph's private arena grows while releases would come
    // from the eager arena.
    FakeDevice dev{kMin};
    Arena eager(256), graph(256);
    Arena::Addr a = 0;
    CHECK(dev.malloc(kMin, &a) == DeviceAlloc::kOk && eager.add_segment(a, kMin));
    dev.log.clear();
    Arena::Span span;
    std::size_t seg = 0;
    CHECK(lmp_hip::grow_and_allocate(graph, eager, 64, kMin, false, dev, &span, &seg) ==
          DeviceAlloc::kOutOfMemory);
    CHECK((dev.log == Log{"malloc 1048576"}) && eager.segment_count() == 1);
    // with release allowed the eager arena's free segment goes back and the
    // new segment joins the graph's arena
    dev.log.clear();
    CHECK(lmp_hip::grow_and_allocate(graph, eager, 64, kMin, true, dev, &span, &seg) ==
          DeviceAlloc::kOk);
    CHECK(eager.segment_count() == 0 && graph.segment_count() == 1 && span.size == 256);
  }
  {
    // A failed wait is an error, and nothing is released after it.
    FakeDevice dev{0};
    dev.fail_sync = true;
    Arena eager(256);
    Arena::Span span;
    std::size_t seg = 0;
    CHECK(lmp_hip::grow_and_allocate(eager, eager, 64, kMin, true, dev, &span, &seg) ==
          DeviceAlloc::kError);
    CHECK((dev.log == std::vector<std::string>{"malloc 1048576", "sync"}));
  }
  {
    // A release that fails is an error, but every other free segment taken
    // from the arena is still released (none is left untracked).
    FakeDevice dev{3 * kMin};
    Arena eager(256);
    Arena::Addr a = 0, b = 0, c = 0;
    CHECK(dev.malloc(kMin, &a) == DeviceAlloc::kOk && eager.add_segment(a, kMin));
    CHECK(dev.malloc(kMin, &b) == DeviceAlloc::kOk && eager.add_segment(b, kMin));
    CHECK(dev.malloc(kMin, &c) == DeviceAlloc::kOk && eager.add_segment(c, kMin));
    dev.fail_free_of = a;
    dev.log.clear();
    Arena::Span span;
    std::size_t seg = 0;
    CHECK(lmp_hip::grow_and_allocate(eager, eager, 64, kMin, true, dev, &span, &seg) ==
          DeviceAlloc::kError);
    CHECK(eager.segment_count() == 0);
    CHECK(dev.live.size() == 1 && dev.live[0].first == a && dev.held == kMin);
    CHECK(dev.log.size() == 5 && dev.log[0] == "malloc 1048576" && dev.log[1] == "sync");
  }
  {
    // A request above the minimum segment gets a segment of its own size.
    FakeDevice dev{64 << 20};
    Arena eager(256);
    Arena::Span span;
    std::size_t seg = 0;
    CHECK(lmp_hip::grow_and_allocate(eager, eager, (5 << 20) + 1, kMin, true, dev, &span, &seg) ==
          DeviceAlloc::kOk);
    CHECK(seg == (std::size_t(5) << 20) + 256 && dev.held == seg);
  }
  return 0;
}

int fastdiv_checks() {
  std::mt19937_64 rng(1);
  const uint32_t special[] = {1, 2, 3, 4, 5, 7, 10, 1000, 1024, 2048, 4096, 16383, 65535,
                              65536, 0x7fffffffu, 0x80000000u, 0x80000001u, 0xfffffffeu,
                              0xffffffffu};
  for (uint32_t d : special) {
    FastDiv f(d);
    const uint32_t ns[] = {0, 1, d - 1, d, d + 1, 0x7fffffffu, 0xfffffffeu, 0xffffffffu};
    for (uint32_t n : ns) CHECK(f.div(n) == n / d);
    for (int i = 0; i < 20000; ++i) {
      uint32_t n = uint32_t(rng());
      CHECK(f.div(n) == n / d);
    }
  }
  for (int i = 0; i < 2000; ++i) {
    uint32_t d = uint32_t(rng() >> (rng() % 32)) | 1u;
    FastDiv f(d);
    for (int j = 0; j < 200; ++j) {
      uint32_t n = uint32_t(rng());
      CHECK(f.div(n) == n / d);
    }
  }
  return 0;
}

int host_copy_checks() {
  lmp_hip::HostCopyPool& pool = lmp_hip::HostCopyPool::get();
  CHECK(pool.threads() >= 1 && pool.threads() <= lmp_hip::kCopyThreads);
  std::mt19937_64 rng(11);
  std::vector<unsigned char> src(24u << 20), dst;
  for (auto& b : src) b = static_cast<unsigned char>(rng());
  const size_t sizes[] = {0, 1, 63, 64, 65, 4096, (1u << 20) - 1, 1u << 20, (1u << 20) + 1,
                          3u << 20, (5u << 20) + 17, (16u << 20) + 12345, 24u << 20};
  for (int round = 0; round < 3; ++round) {
    for (size_t n : sizes) {
      const size_t off = n < src.size() ? rng() % (src.size() - n + 1) : 0;
      dst.assign(n + 32, 0xAB);
      pool.copy(dst.data() + 16, src.data() + off, n);
      CHECK(std::memcmp(dst.data() + 16, src.data() + off, n) == 0);
      for (int i = 0; i < 16; ++i) CHECK(dst[i] == 0xAB && dst[n + 16 + i] == 0xAB);
    }
  }
  return 0;
}

int main() {
  if (arena_checks()) return 1;
  if (host_copy_checks()) return 1;
  if (growth_policy_checks()) return 1;
  if (fastdiv_checks()) return 1;
  std::printf("host checks ok\n");
  return 0;
}
