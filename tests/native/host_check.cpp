// Host-only checks of the backend's CPU-side logic: the caching arena
// (best fit, split, coalesce, segment release, unknown-address rejection)
// and the magic-number divider.  Built and run by tests/test_host_native.py
// with g++; no GPU involved.
#include <cassert>
#include <cstdio>
#include <random>

#include "arena.hpp"
#include "fastdiv.hpp"

using lmp_hip::Arena;
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

int main() {
  if (arena_checks()) return 1;
  if (fastdiv_checks()) return 1;
  std::printf("host checks ok\n");
  return 0;
}
