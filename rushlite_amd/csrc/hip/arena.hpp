// Host-only best-fit arena behind lmp_rt_malloc/lmp_rt_free.
//
// Policy follows Lamp3's CUDA caching allocator (BlockArena,
// csrc/src/tensor/cuda/allocator_core.hpp:33-207, allocator.cu:17-128):
// 256-byte aligned best-fit suballocation from large device segments, split
// on allocate, coalesce with free neighbours of the same segment on free, and
// hand back segments that are entirely free when the device runs out.
//
// The data structure is this file's own: blocks live in one address-ordered
// map (neighbours are the previous/next map entries), free blocks are indexed
// by (size, address) in an ordered set, so "best fit" is the first free entry
// not smaller than the request and ties go to the lowest address.  Nothing
// here touches the GPU; addresses are plain integers so tests can drive it
// with synthetic segments.
#pragma once

#include <cstddef>
#include <cstdint>
#include <iterator>
#include <map>
#include <optional>
#include <set>
#include <utility>
#include <vector>

namespace lmp_hip {

class Arena {
 public:
  using Addr = std::uintptr_t;

  struct Span {
    Addr addr = 0;
    std::size_t size = 0;
  };

  explicit Arena(std::size_t alignment) : align_(alignment) {}

  std::size_t alignment() const { return align_; }

  std::size_t round_up(std::size_t n) const {
    return (n + align_ - 1) / align_ * align_;
  }

  // Register [addr, addr+size) as a new segment made of one free block.
  // Returns false if the span is misaligned, empty or overlaps a segment.
  bool add_segment(Addr addr, std::size_t size) {
    if (addr == 0 || size == 0 || addr % align_ != 0 || size % align_ != 0)
      return false;
    auto next = segments_.lower_bound(addr);
    if (next != segments_.end() && next->first < addr + size) return false;
    if (next != segments_.begin()) {
      auto prev = std::prev(next);
      if (prev->first + prev->second > addr) return false;
    }
    segments_.emplace(addr, size);
    blocks_.emplace(addr, Block{size, addr, false});
    free_.emplace(size, addr);
    reserved_ += size;
    return true;
  }

  // Best-fit allocation; nullopt when no free block is large enough.
  // A zero-byte request yields a null span.
  std::optional<Span> allocate(std::size_t bytes) {
    if (bytes == 0) return Span{};
    const std::size_t need = round_up(bytes);
    auto fit = free_.lower_bound({need, 0});
    if (fit == free_.end()) return std::nullopt;
    const Addr addr = fit->second;
    free_.erase(fit);
    Block& blk = blocks_.at(addr);
    if (blk.size > need) {
      const Addr rest = addr + need;
      const std::size_t rest_size = blk.size - need;
      blocks_.emplace(rest, Block{rest_size, blk.segment, false});
      free_.emplace(rest_size, rest);
      blk.size = need;
    }
    blk.used = true;
    in_use_ += need;
    return Span{addr, need};
  }

  // Release a block returned by allocate().  Unknown or already-free
  // addresses return false and change nothing.
  bool release(Addr addr) {
    if (addr == 0) return true;
    auto it = blocks_.find(addr);
    if (it == blocks_.end() || !it->second.used) return false;
    it->second.used = false;
    in_use_ -= it->second.size;
    // merge with the following block
    auto nxt = std::next(it);
    if (nxt != blocks_.end() && !nxt->second.used &&
        nxt->second.segment == it->second.segment &&
        it->first + it->second.size == nxt->first) {
      free_.erase({nxt->second.size, nxt->first});
      it->second.size += nxt->second.size;
      blocks_.erase(nxt);
    }
    // merge into the preceding block
    if (it != blocks_.begin()) {
      auto prv = std::prev(it);
      if (!prv->second.used && prv->second.segment == it->second.segment &&
          prv->first + prv->second.size == it->first) {
        free_.erase({prv->second.size, prv->first});
        prv->second.size += it->second.size;
        blocks_.erase(it);
        it = prv;
      }
    }
    free_.emplace(it->second.size, it->first);
    return true;
  }

  // Remove every segment that is one free block and return their spans so
  // the caller can give the memory back to the device runtime.
  std::vector<Span> take_free_segments() {
    std::vector<Span> out;
    for (auto seg = segments_.begin(); seg != segments_.end();) {
      auto blk = blocks_.find(seg->first);
      if (blk != blocks_.end() && !blk->second.used &&
          blk->second.size == seg->second) {
        free_.erase({blk->second.size, blk->first});
        blocks_.erase(blk);
        out.push_back({seg->first, seg->second});
        reserved_ -= seg->second;
        seg = segments_.erase(seg);
      } else {
        ++seg;
      }
    }
    return out;
  }

  std::size_t reserved_bytes() const { return reserved_; }
  std::size_t in_use_bytes() const { return in_use_; }
  std::size_t segment_count() const { return segments_.size(); }
  std::size_t free_block_count() const { return free_.size(); }
  std::size_t block_count() const { return blocks_.size(); }

 private:
  struct Block {
    std::size_t size;
    Addr segment;  // base address of the owning segment
    bool used;
  };

  std::size_t align_;
  std::size_t reserved_ = 0;
  std::size_t in_use_ = 0;
  std::map<Addr, std::size_t> segments_;          // base -> size
  std::map<Addr, Block> blocks_;                  // every block, by address
  std::set<std::pair<std::size_t, Addr>> free_;   // (size, addr) of free ones
};

// Result of asking the device for memory.
enum class DeviceAlloc { kOk, kOutOfMemory, kError };

// What happens when no free block of an arena can serve a request
// (allocator.cu:101-125): ask the device for a new segment of
// max(min_segment, the rounded request); if the device is out of memory and
// `may_release` allows it (not while a graph is being captured), wait for the
// queued work so no cached block is still in use, give every wholly free
// segment of `cache` back to the device, and ask once more.  The new segment
// joins `target` (the eager arena, or a graph's private one) and the request
// is served from it.  Dev supplies the device side:
//   DeviceAlloc malloc(std::size_t bytes, Arena::Addr* base);
//   bool sync();                         // false: the wait itself failed
//   bool free(Arena::Addr base);         // false: the release failed
// Returns kOk with *out set, kOutOfMemory when the device refused even after
// the release, or kError when a device call failed or the segment it returned
// cannot be added (that segment goes back to the device); *segment gets the
// size asked for.
template <class Dev>
DeviceAlloc grow_and_allocate(Arena& target, Arena& cache, std::size_t bytes,
                              std::size_t min_segment, bool may_release, Dev& dev,
                              Arena::Span* out, std::size_t* segment) {
  const std::size_t need = target.round_up(bytes);
  const std::size_t seg = need > min_segment ? need : min_segment;
  *segment = seg;
  Arena::Addr base = 0;
  DeviceAlloc st = dev.malloc(seg, &base);
  if (st == DeviceAlloc::kOutOfMemory && may_release) {
    if (!dev.sync()) return DeviceAlloc::kError;
    // Every taken segment is released even past a failed release: they are
    // no longer tracked by the arena, so one skipped here would leak.
    bool released = true;
    for (const Arena::Span& s : cache.take_free_segments())
      released = dev.free(s.addr) && released;
    if (!released) return DeviceAlloc::kError;
    st = dev.malloc(seg, &base);
  }
  if (st != DeviceAlloc::kOk) return st;
  if (!target.add_segment(base, seg)) {
    (void)dev.free(base);
    return DeviceAlloc::kError;
  }
  auto span = target.allocate(bytes);
  if (!span) return DeviceAlloc::kError;
  *out = *span;
  return DeviceAlloc::kOk;
}

}  // namespace lmp_hip
