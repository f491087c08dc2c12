// Internal helpers shared by the HIP translation units of liblmp_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "fastdiv.hpp"
#include "lmp_hip.h"

namespace lmp_hip {

// Thread-local message behind lmp_rt_last_error().
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);

// Counts every kernel the library launches (lmp_rt_kernel_launch_count).
void count_kernel_launch();

// Runtime state of the library: one device, one in-order stream.
struct Runtime {
  int device = -1;
  hipStream_t stream = nullptr;
  int cu_count = 0;
  int max_threads_per_cu = 2048;
  size_t lds_per_cu = 0;
  // Device address of the bound device's copy of the no-allocation
  // workspace (LMP_NOALLOC_SCRATCH_BYTES), looked up once at set-up; null
  // with the reason in noalloc_error when the lookup failed.
  void* noalloc_scratch = nullptr;
  std::string noalloc_error;
};

// Initialise lazily on device 0 when a kernel entry runs before lmp_rt_init.
// Returns nullptr (with the error set) when no device is usable.
Runtime* runtime();

// Operands at least as large as the 256 MB memory-side cache (MALL) are read
// with the nontemporal hint: they cannot stay in that cache between uses, and
// reads that do not allocate there stream faster (on MI355X a cold 256 MiB
// read + write 84.4 -> 81.5 us; a 1 GiB read 186 -> 165 us in a plain probe).
// Smaller operands may still be there from the kernel that wrote them (a warm
// 256 MiB re-read: 64.7 us with ordinary loads, 78.5 us nontemporal), so they
// keep ordinary loads.
constexpr uint64_t kStreamBytes = uint64_t(256) << 20;

// Outputs of more than half the MALL are written with the nontemporal hint,
// smaller ones with ordinary stores: a kernel that reads an output soon after
// it is written finds an ordinary-stored one in the MALL (a producer and its
// consumer over 64 MiB operands on MI355X: 56.8 -> 46.5 us; 128 MiB: 110 ->
// 86 us), while from 192 MiB on the nontemporal stores are faster (164 vs
// 173 us; 256 MiB: 219 vs 227 us).
constexpr uint64_t kStreamStoreBytes = uint64_t(128) << 20;

// GEMM extents (M, N, K) and leading dimensions stay below 2^31 - 4096, so
// that every tile origin, fragment index and K-loop step (an extent plus at
// most a few thousand) still fits the kernels' int arithmetic.
constexpr size_t kGemmMaxExtent = (size_t(1) << 31) - 4096;

// Scratch allocation for kernels that need a workspace (split-K partials,
// two-pass reductions).  Memory comes from the pool and is returned to it
// by the matching release; ordering on the single stream makes reuse safe.
void* scratch_alloc(size_t bytes);
void scratch_free(void* ptr);

inline size_t dtype_size(int dtype) {
  switch (dtype) {
    case LMP_BOOL: return 1;
    case LMP_INT16: return 2;
    case LMP_INT32: return 4;
    case LMP_INT64: return 8;
    case LMP_FLOAT32: return 4;
    case LMP_FLOAT64: return 8;
    default: return 0;
  }
}

inline const char* dtype_name(int dtype) {
  switch (dtype) {
    case LMP_BOOL: return "Bool";
    case LMP_INT16: return "Int16";
    case LMP_INT32: return "Int32";
    case LMP_INT64: return "Int64";
    case LMP_FLOAT32: return "Float32";
    case LMP_FLOAT64: return "Float64";
    default: return "Unknown";
  }
}

#define LMP_HIP_TRY(expr)                                                   \
  do {                                                                      \
    hipError_t _e = (expr);                                                 \
    if (_e != hipSuccess)                                                   \
      return ::lmp_hip::fail(LMP_ERR_RUNTIME,                               \
                             std::string(#expr) + ": " + hipGetErrorString(_e)); \
  } while (0)

// Check the launch that was just issued (every launch site issues exactly
// one launch before its check) and count it.
#define LMP_LAUNCH_CHECK(name)                                              \
  do {                                                                      \
    hipError_t _e = hipGetLastError();                                      \
    if (_e != hipSuccess)                                                   \
      return ::lmp_hip::fail(LMP_ERR_RUNTIME,                               \
                             std::string("launch of ") + (name) + ": " +    \
                                 hipGetErrorString(_e));                    \
    ::lmp_hip::count_kernel_launch();                                       \
  } while (0)

#define LMP_RUNTIME_OR_FAIL(rt)                                             \
  ::lmp_hip::Runtime* rt = ::lmp_hip::runtime();                            \
  if (!rt) return LMP_ERR_RUNTIME

}  // namespace lmp_hip
