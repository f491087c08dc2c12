// Runtime half of the C ABI: device selection, the pooled allocator, copies,
// synchronisation and timing events.  These are the only hip* runtime calls
// of the backend apart from kernel launches and the hipRTC module loader.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "arena.hpp"
#include "common.hpp"
#include "host_copy.hpp"

// Workspace of the no-allocation entry point (lmp_k_gemm_f32_noalloc): a
// fixed device array, one copy on each device the library's code object is
// loaded on, held until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host the name is only a stand-in): set-up looks
// up the device's copy with hipGetSymbolAddress and keeps that address.
static __device__ __align__(256) float scratch[LMP_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace lmp_hip {

namespace {

thread_local std::string t_error;

// Segment granularity: with 288 GB of HBM per MI355X a large minimum keeps the
// segment count low; requests above it get a segment of their own size.
constexpr size_t kAlign = 256;
constexpr size_t kMinSegment = 128ull << 20;

// Memory of one captured graph.  Every block allocated while the graph is
// captured comes from here and returns here when freed, so no eager
// allocation can reuse an address the graph's replays write.  Segments go back
// to HIP once the graph is destroyed and the last block is freed.
struct GraphPool {
  Arena arena{kAlign};
  bool dead = false;
};

struct Pool {
  std::mutex mu;
  Arena arena{kAlign};
  std::vector<std::unique_ptr<GraphPool>> graph_pools;
  GraphPool* capturing = nullptr;  // allocation target during a graph capture
  uint64_t allocs = 0;
  uint64_t device_mallocs = 0;
};

// A captured, instantiated graph (the opaque handle of lmp_rt_graph_*).
struct GraphHandle {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  GraphPool* pool = nullptr;
};

Pool& pool() {
  // Immortal: tensors held by static objects may be freed during exit.
  static Pool* p = new Pool();
  return *p;
}

std::mutex g_init_mu;
Runtime g_rt;
bool g_ready = false;

int init_locked(int device) {
  if (g_ready) {
    if (device != g_rt.device)
      return fail(LMP_ERR_INVALID,
                  "lmp_rt_init: library already bound to device " +
                      std::to_string(g_rt.device));
    return LMP_OK;
  }
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(LMP_ERR_RUNTIME,
                std::string("no HIP device available: ") +
                    (e == hipSuccess ? "device count is 0"
                                     : hipGetErrorString(e)));
  if (device < 0 || device >= count)
    return fail(LMP_ERR_INVALID, "lmp_rt_init: device index out of range");
  LMP_HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  LMP_HIP_TRY(hipGetDeviceProperties(&prop, device));
  // Default priority: the stream is created without a priority argument.
  LMP_HIP_TRY(hipStreamCreateWithFlags(&g_rt.stream, hipStreamNonBlocking));
  g_rt.device = device;
  g_rt.cu_count = prop.multiProcessorCount;
  g_rt.max_threads_per_cu = prop.maxThreadsPerMultiProcessor;
  g_rt.lds_per_cu = prop.maxSharedMemoryPerMultiProcessor;
  // The bound device's copy of the no-allocation workspace (this device is
  // current).  A failed lookup leaves only that entry point unusable: it
  // reports the reason; every other entry point works as before.
  void* ws = nullptr;
  const hipError_t we = hipGetSymbolAddress(&ws, HIP_SYMBOL(scratch));
  if (we == hipSuccess && ws) {
    g_rt.noalloc_scratch = ws;
  } else {
    g_rt.noalloc_error = std::string("hipGetSymbolAddress(scratch): ") +
                         (we == hipSuccess ? "null address" : hipGetErrorString(we));
    (void)hipGetLastError();
  }
  g_ready = true;
  return LMP_OK;
}

// The device side of Arena's growth policy: hipMalloc, a stream wait and
// hipFree, keeping the text of the first failure.
struct HipSegments {
  std::string error;
  DeviceAlloc malloc(size_t bytes, Arena::Addr* base) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e == hipSuccess) {
      *base = reinterpret_cast<Arena::Addr>(p);
      return DeviceAlloc::kOk;
    }
    (void)hipGetLastError();
    error = "hipMalloc of " + std::to_string(bytes) + " bytes failed: " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation ? DeviceAlloc::kOutOfMemory
                                                                     : DeviceAlloc::kError;
  }
  bool sync() {
    const hipError_t e = hipStreamSynchronize(g_rt.stream);
    if (e != hipSuccess) error = std::string("hipStreamSynchronize: ") + hipGetErrorString(e);
    return e == hipSuccess;
  }
  bool free(Arena::Addr base) {
    const hipError_t e = hipFree(reinterpret_cast<void*>(base));
    if (e != hipSuccess) error = std::string("hipFree: ") + hipGetErrorString(e);
    return e == hipSuccess;
  }
};

int grow_and_allocate(Pool& p, Arena& arena, size_t bytes, void** out) {
  HipSegments dev;
  Arena::Span span;
  size_t seg = 0;
  // The release-and-retry path synchronises the stream, which a capture forbids.
  const DeviceAlloc st = lmp_hip::grow_and_allocate(arena, p.arena, bytes, kMinSegment,
                                                    !p.capturing, dev, &span, &seg);
  if (st == DeviceAlloc::kOk) {
    ++p.device_mallocs;
    *out = reinterpret_cast<void*>(span.addr);
    return LMP_OK;
  }
  if (st == DeviceAlloc::kOutOfMemory) return fail(LMP_ERR_OOM, dev.error);
  return fail(LMP_ERR_RUNTIME,
              dev.error.empty() ? std::string("allocator: the new segment of ") + std::to_string(seg) +
                                      " bytes cannot serve the request"
                                : dev.error);
}

// Hand the segments of destroyed graphs whose blocks are all freed back to
// HIP.  Needs an idle stream (a replay may still be running), so it never runs
// during a capture.  Called with p.mu held.
int release_dead_pools(Pool& p) {
  if (p.capturing) return LMP_OK;
  bool any = false;
  for (const auto& gp : p.graph_pools) any |= gp->dead && gp->arena.in_use_bytes() == 0;
  if (!any) return LMP_OK;
  LMP_HIP_TRY(hipStreamSynchronize(g_rt.stream));
  for (auto it = p.graph_pools.begin(); it != p.graph_pools.end();) {
    GraphPool& gp = **it;
    if (gp.dead && gp.arena.in_use_bytes() == 0) {
      for (const Arena::Span& s : gp.arena.take_free_segments())
        LMP_HIP_TRY(hipFree(reinterpret_cast<void*>(s.addr)));
      it = p.graph_pools.erase(it);
    } else {
      ++it;
    }
  }
  return LMP_OK;
}

bool capturing() {
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  return p.capturing != nullptr;
}

#define LMP_NOT_WHILE_CAPTURING(what)                                          \
  do {                                                                         \
    if (capturing())                                                           \
      return fail(LMP_ERR_INVALID, std::string(what) +                         \
                                       ": not allowed while a graph is being " \
                                       "captured");                            \
  } while (0)

// ------------------------------------------------------------- staged copies
//
// Large host <-> device copies run through two pinned staging buffers: the DMA
// engine moves one chunk between HBM and pinned memory while host threads copy
// the neighbouring chunk between pinned memory and the caller's pageable
// buffer.  HIP's own pageable path does the two halves one after the other on
// one host thread; on an MI355X box: pinned DMA 57 GB/s each way, pageable
// hipMemcpy 29 GB/s up and 4-18 GB/s down (new or reused host memory), one
// host thread copying into new (faulting) memory 4.5 GB/s, eight 22 GB/s.
constexpr size_t kStageChunk = size_t(16) << 20;
constexpr size_t kStagedMin = size_t(4) << 20;  // smaller copies go direct

struct Staging {
  std::mutex mu;  // one staged copy at a time
  void* buf[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int state = 0;  // 0 not yet set up, 1 ready, -1 unavailable (copies go direct)
};

Staging& staging() {
  static Staging* s = new Staging();  // immortal, like the pool
  return *s;
}

// With s.mu held.  A failed set-up leaves the direct path in use.
bool staging_ready(Staging& s) {
  if (s.state == 0) {
    s.state = -1;
    for (int i = 0; i < 2; ++i) {
      if (hipHostMalloc(&s.buf[i], kStageChunk, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&s.done[i], hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return false;
      }
    }
    s.state = 1;
  }
  return s.state == 1;
}

// Device -> pageable host in chunks: DMA of chunk c + 1 into one staging
// buffer overlaps the host threads' copy of chunk c out of the other.
int staged_d2h(Runtime* rt, Staging& st, char* dst, const char* src, size_t bytes) {
  const size_t chunks = (bytes + kStageChunk - 1) / kStageChunk;
  auto len = [&](size_t c) { return std::min(kStageChunk, bytes - c * kStageChunk); };
  auto issue = [&](size_t c) -> hipError_t {
    hipError_t e = hipMemcpyAsync(st.buf[c & 1], src + c * kStageChunk, len(c),
                                  hipMemcpyDeviceToHost, rt->stream);
    return e != hipSuccess ? e : hipEventRecord(st.done[c & 1], rt->stream);
  };
  hipError_t e = issue(0);
  if (e == hipSuccess && chunks > 1) e = issue(1);
  for (size_t c = 0; c < chunks && e == hipSuccess; ++c) {
    e = hipEventSynchronize(st.done[c & 1]);
    if (e != hipSuccess) break;
    HostCopyPool::get().copy(dst + c * kStageChunk, st.buf[c & 1], len(c));
    if (c + 2 < chunks) e = issue(c + 2);
  }
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(rt->stream);  // no DMA left writing the staging buffers
    return fail(LMP_ERR_RUNTIME, std::string("memcpy_d2h (staged): ") + hipGetErrorString(e));
  }
  return LMP_OK;
}

// Pageable host -> device: the host threads fill one staging buffer while the
// DMA engine empties the other; returns once every chunk has landed.
int staged_h2d(Runtime* rt, Staging& st, char* dst, const char* src, size_t bytes) {
  const size_t chunks = (bytes + kStageChunk - 1) / kStageChunk;
  hipError_t e = hipSuccess;
  for (size_t c = 0; c < chunks && e == hipSuccess; ++c) {
    const size_t n = std::min(kStageChunk, bytes - c * kStageChunk);
    if (c >= 2) {
      e = hipEventSynchronize(st.done[c & 1]);  // its previous chunk has been read
      if (e != hipSuccess) break;
    }
    HostCopyPool::get().copy(st.buf[c & 1], src + c * kStageChunk, n);
    e = hipMemcpyAsync(dst + c * kStageChunk, st.buf[c & 1], n, hipMemcpyHostToDevice,
                       rt->stream);
    if (e == hipSuccess) e = hipEventRecord(st.done[c & 1], rt->stream);
  }
  const hipError_t se = hipStreamSynchronize(rt->stream);
  if (e == hipSuccess) e = se;
  if (e != hipSuccess)
    return fail(LMP_ERR_RUNTIME, std::string("memcpy_h2d (staged): ") + hipGetErrorString(e));
  return LMP_OK;
}

}  // namespace

void set_error(const std::string& msg) { t_error = msg; }

int fail(int status, const std::string& msg) {
  t_error = msg;
  return status;
}

namespace {
std::atomic<uint64_t> g_kernel_launches{0};
}  // namespace

void count_kernel_launch() { g_kernel_launches.fetch_add(1, std::memory_order_relaxed); }

Runtime* runtime() {
  std::lock_guard<std::mutex> lock(g_init_mu);
  if (!g_ready && init_locked(0) != LMP_OK) return nullptr;
  return &g_rt;
}

void* scratch_alloc(size_t bytes) {
  void* p = nullptr;
  if (lmp_rt_malloc(&p, bytes) != LMP_OK) return nullptr;
  return p;
}

void scratch_free(void* ptr) { (void)lmp_rt_free(ptr); }

}  // namespace lmp_hip

using namespace lmp_hip;

extern "C" {

int lmp_rt_abi_version(void) { return LMP_HIP_ABI_VERSION; }

const char* lmp_rt_last_error(void) { return t_error.c_str(); }

int lmp_rt_init(int device) {
  std::lock_guard<std::mutex> lock(g_init_mu);
  return init_locked(device);
}

int lmp_rt_device_count(int* count) {
  if (!count) return fail(LMP_ERR_INVALID, "null count");
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e != hipSuccess) {
    *count = 0;
    (void)hipGetLastError();
  }
  return LMP_OK;
}

int lmp_rt_device_info(lmp_rt_info* info) {
  if (!info) return fail(LMP_ERR_INVALID, "null info");
  LMP_RUNTIME_OR_FAIL(rt);
  hipDeviceProp_t prop;
  LMP_HIP_TRY(hipGetDeviceProperties(&prop, rt->device));
  std::memset(info, 0, sizeof(*info));
  info->device = rt->device;
  info->cu_count = prop.multiProcessorCount;
  info->simd_per_cu = 4;
  info->wave_size = prop.warpSize;
  info->lds_bytes_per_cu = static_cast<int64_t>(prop.maxSharedMemoryPerMultiProcessor);
  info->total_mem_bytes = static_cast<int64_t>(prop.totalGlobalMem);
  info->clock_khz = prop.clockRate;
  info->mem_clock_khz = prop.memoryClockRate;
  info->mem_bus_width = prop.memoryBusWidth;
  std::strncpy(info->arch, prop.gcnArchName, sizeof(info->arch) - 1);
  std::strncpy(info->name, prop.name, sizeof(info->name) - 1);
  return LMP_OK;
}

int lmp_rt_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(LMP_ERR_INVALID, "lmp_rt_malloc: null out pointer");
  *ptr = nullptr;
  if (bytes == 0) return LMP_OK;
  LMP_RUNTIME_OR_FAIL(rt);
  (void)rt;
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  ++p.allocs;
  Arena& arena = p.capturing ? p.capturing->arena : p.arena;
  if (auto span = arena.allocate(bytes)) {
    *ptr = reinterpret_cast<void*>(span->addr);
    return LMP_OK;
  }
  return grow_and_allocate(p, arena, bytes, ptr);
}

int lmp_rt_free(void* ptr) {
  if (!ptr) return LMP_OK;
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  const auto addr = reinterpret_cast<Arena::Addr>(ptr);
  if (p.arena.release(addr)) return LMP_OK;
  for (const auto& gp : p.graph_pools) {
    if (gp->arena.release(addr)) return gp->dead ? release_dead_pools(p) : LMP_OK;
  }
  return fail(LMP_ERR_INVALID, "lmp_rt_free: pointer not owned by the pool");
}

int lmp_rt_empty_cache(void) {
  LMP_RUNTIME_OR_FAIL(rt);
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  if (p.capturing)
    return fail(LMP_ERR_INVALID, "lmp_rt_empty_cache: not allowed while a graph is being captured");
  LMP_HIP_TRY(hipStreamSynchronize(rt->stream));
  for (const Arena::Span& s : p.arena.take_free_segments())
    LMP_HIP_TRY(hipFree(reinterpret_cast<void*>(s.addr)));
  return release_dead_pools(p);
}

int lmp_rt_kernel_launch_count(uint64_t* count) {
  if (!count) return fail(LMP_ERR_INVALID, "null count");
  *count = g_kernel_launches.load(std::memory_order_relaxed);
  return LMP_OK;
}

int lmp_rt_pool_stats_get(lmp_rt_pool_stats* stats) {
  if (!stats) return fail(LMP_ERR_INVALID, "null stats");
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  stats->reserved_bytes = p.arena.reserved_bytes();
  stats->allocated_bytes = p.arena.in_use_bytes();
  stats->segments = p.arena.segment_count();
  stats->allocs = p.allocs;
  stats->device_mallocs = p.device_mallocs;
  return LMP_OK;
}

int lmp_rt_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return LMP_OK;
  if (!dst || !src) return fail(LMP_ERR_INVALID, "memcpy_h2d: null pointer");
  LMP_NOT_WHILE_CAPTURING("memcpy_h2d");
  LMP_RUNTIME_OR_FAIL(rt);
  if (bytes >= kStagedMin) {
    Staging& st = staging();
    std::lock_guard<std::mutex> lock(st.mu);
    if (staging_ready(st))
      return staged_h2d(rt, st, static_cast<char*>(dst), static_cast<const char*>(src), bytes);
  }
  LMP_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, rt->stream));
  // The source may be pageable memory the caller reuses right away.
  LMP_HIP_TRY(hipStreamSynchronize(rt->stream));
  return LMP_OK;
}

int lmp_rt_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return LMP_OK;
  if (!dst || !src) return fail(LMP_ERR_INVALID, "memcpy_d2h: null pointer");
  LMP_NOT_WHILE_CAPTURING("memcpy_d2h");
  LMP_RUNTIME_OR_FAIL(rt);
  if (bytes >= kStagedMin) {
    Staging& st = staging();
    std::lock_guard<std::mutex> lock(st.mu);
    if (staging_ready(st))
      return staged_d2h(rt, st, static_cast<char*>(dst), static_cast<const char*>(src), bytes);
  }
  LMP_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, rt->stream));
  LMP_HIP_TRY(hipStreamSynchronize(rt->stream));
  return LMP_OK;
}

int lmp_rt_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return LMP_OK;
  if (!dst || !src) return fail(LMP_ERR_INVALID, "memcpy_d2d: null pointer");
  LMP_RUNTIME_OR_FAIL(rt);
  LMP_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, rt->stream));
  return LMP_OK;
}

int lmp_rt_synchronize(void) {
  LMP_NOT_WHILE_CAPTURING("synchronize");
  LMP_RUNTIME_OR_FAIL(rt);
  LMP_HIP_TRY(hipStreamSynchronize(rt->stream));
  return LMP_OK;
}

void* lmp_rt_stream(void) {
  Runtime* rt = runtime();
  return rt ? static_cast<void*>(rt->stream) : nullptr;
}

int lmp_rt_event_create(void** event) {
  if (!event) return fail(LMP_ERR_INVALID, "null event");
  LMP_RUNTIME_OR_FAIL(rt);
  (void)rt;
  hipEvent_t e;
  LMP_HIP_TRY(hipEventCreate(&e));
  *event = e;
  return LMP_OK;
}

int lmp_rt_event_record(void* event) {
  if (!event) return fail(LMP_ERR_INVALID, "null event");
  LMP_RUNTIME_OR_FAIL(rt);
  LMP_HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(event), rt->stream));
  return LMP_OK;
}

int lmp_rt_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (!start || !stop || !ms) return fail(LMP_ERR_INVALID, "null argument");
  LMP_NOT_WHILE_CAPTURING("event_elapsed_ms");
  LMP_HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  LMP_HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                  static_cast<hipEvent_t>(stop)));
  return LMP_OK;
}

int lmp_rt_event_destroy(void* event) {
  if (!event) return LMP_OK;
  LMP_HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return LMP_OK;
}

int lmp_rt_graph_begin(void) {
  LMP_RUNTIME_OR_FAIL(rt);
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  if (p.capturing) return fail(LMP_ERR_INVALID, "graph_begin: a capture is already open");
  // Eager work queued before the capture runs now, outside the graph.
  LMP_HIP_TRY(hipStreamSynchronize(rt->stream));
  auto gp = std::make_unique<GraphPool>();
  // Relaxed mode: pool growth (hipMalloc) stays legal inside the capture.
  hipError_t e = hipStreamBeginCapture(rt->stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(LMP_ERR_RUNTIME, std::string("hipStreamBeginCapture: ") + hipGetErrorString(e));
  }
  p.capturing = gp.get();
  p.graph_pools.push_back(std::move(gp));
  return LMP_OK;
}

int lmp_rt_graph_end(void** graph) {
  if (!graph) return fail(LMP_ERR_INVALID, "graph_end: null out pointer");
  *graph = nullptr;
  LMP_RUNTIME_OR_FAIL(rt);
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  if (!p.capturing) return fail(LMP_ERR_INVALID, "graph_end: no capture is open");
  GraphPool* gp = p.capturing;
  p.capturing = nullptr;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(rt->stream, &g);
  hipGraphExec_t exec = nullptr;
  if (e == hipSuccess) e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (g) (void)hipGraphDestroy(g);
    gp->dead = true;  // blocks still held by tensors keep it until freed
    return fail(LMP_ERR_RUNTIME, std::string("graph capture failed: ") + hipGetErrorString(e));
  }
  *graph = new GraphHandle{g, exec, gp};
  return LMP_OK;
}

int lmp_rt_graph_abort(void) {
  LMP_RUNTIME_OR_FAIL(rt);
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  if (!p.capturing) return LMP_OK;
  p.capturing->dead = true;
  p.capturing = nullptr;
  hipGraph_t g = nullptr;
  (void)hipStreamEndCapture(rt->stream, &g);
  (void)hipGetLastError();
  if (g) (void)hipGraphDestroy(g);
  return LMP_OK;
}

int lmp_rt_graph_launch(void* graph) {
  if (!graph) return fail(LMP_ERR_INVALID, "graph_launch: null graph");
  LMP_NOT_WHILE_CAPTURING("graph_launch");
  LMP_RUNTIME_OR_FAIL(rt);
  LMP_HIP_TRY(hipGraphLaunch(static_cast<GraphHandle*>(graph)->exec, rt->stream));
  return LMP_OK;
}

int lmp_rt_graph_destroy(void* graph) {
  if (!graph) return LMP_OK;
  LMP_NOT_WHILE_CAPTURING("graph_destroy");
  LMP_RUNTIME_OR_FAIL(rt);
  auto* h = static_cast<GraphHandle*>(graph);
  LMP_HIP_TRY(hipStreamSynchronize(rt->stream));
  LMP_HIP_TRY(hipGraphExecDestroy(h->exec));
  LMP_HIP_TRY(hipGraphDestroy(h->graph));
  Pool& p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  h->pool->dead = true;
  delete h;
  return release_dead_pools(p);
}

}  // extern "C"
