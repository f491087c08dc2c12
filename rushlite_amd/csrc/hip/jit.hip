// hipRTC module cache for the lazy-fusion backend (replaces the NVRTC cache
// of nvrtc_backend.cpp:19-128).  The caller keys modules by a 64-bit hash of
// the captured graph's structure, so a repeated graph costs one map lookup
// and no source generation.  Sources compile for the running device's exact
// gcnArchName (gfx950 on MI355X) with -O3 and -ffp-contract=off: eager Lamp3
// rounds after every op, so a fused a*a+b must not become an FMA.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace lmp_hip {
namespace {

struct JitKernel {
  hipModule_t module = nullptr;
  hipFunction_t fn = nullptr;
  std::string name;
};

struct JitCache {
  std::mutex mu;
  std::unordered_map<uint64_t, std::unique_ptr<JitKernel>> map;
  uint64_t compiled = 0;
  std::string arch;
};

JitCache& cache() {
  static JitCache* c = new JitCache();
  return *c;
}

std::string device_arch(Runtime* rt) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, rt->device) != hipSuccess) return "gfx950";
  return prop.gcnArchName;
}

}  // namespace
}  // namespace lmp_hip

using namespace lmp_hip;

extern "C" {

int lmp_jit_lookup(uint64_t key, void** handle) {
  if (!handle) return fail(LMP_ERR_INVALID, "lmp_jit_lookup: null handle");
  JitCache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  auto it = c.map.find(key);
  if (it == c.map.end()) {
    *handle = nullptr;
    return LMP_ERR_INVALID;
  }
  *handle = it->second.get();
  return LMP_OK;
}

int lmp_jit_compile(uint64_t key, const char* source, const char* kernel_name,
                    void** handle) {
  if (!handle || !source || !kernel_name)
    return fail(LMP_ERR_INVALID, "lmp_jit_compile: null argument");
  LMP_RUNTIME_OR_FAIL(rt);
  JitCache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  auto it = c.map.find(key);
  if (it != c.map.end()) {
    *handle = it->second.get();
    return LMP_OK;
  }
  if (c.arch.empty()) c.arch = device_arch(rt);

  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, "lmp_fused.hip", 0,
                                       nullptr, nullptr);
  if (r != HIPRTC_SUCCESS)
    return fail(LMP_ERR_JIT, std::string("hiprtcCreateProgram: ") +
                                 hiprtcGetErrorString(r));
  const std::string arch_opt = "--offload-arch=" + c.arch;
  // Packed fp32 VALU forms stay disabled, as for the precompiled kernels.
  const char* opts[] = {arch_opt.c_str(), "-O3",      "-ffp-contract=off",
                        "-std=c++17",     "-Xclang",  "-target-feature",
                        "-Xclang",        "-packed-fp32-ops"};
  r = hiprtcCompileProgram(prog, 8, opts);
  if (r != HIPRTC_SUCCESS) {
    size_t log_size = 0;
    hiprtcGetProgramLogSize(prog, &log_size);
    std::string log(log_size, '\0');
    if (log_size) hiprtcGetProgramLog(prog, log.data());
    hiprtcDestroyProgram(&prog);
    return fail(LMP_ERR_JIT, std::string("hipRTC compile failed: ") +
                                 hiprtcGetErrorString(r) + "\n" + log +
                                 "\n--- generated source ---\n" + source);
  }
  size_t code_size = 0;
  hiprtcGetCodeSize(prog, &code_size);
  std::vector<char> code(code_size);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);

  auto k = std::make_unique<JitKernel>();
  k->name = kernel_name;
  hipError_t e = hipModuleLoadData(&k->module, code.data());
  if (e != hipSuccess)
    return fail(LMP_ERR_JIT, std::string("hipModuleLoadData: ") + hipGetErrorString(e));
  e = hipModuleGetFunction(&k->fn, k->module, kernel_name);
  if (e != hipSuccess) {
    (void)hipModuleUnload(k->module);
    return fail(LMP_ERR_JIT, std::string("hipModuleGetFunction(") + kernel_name +
                                 "): " + hipGetErrorString(e));
  }
  *handle = k.get();
  c.map.emplace(key, std::move(k));
  ++c.compiled;
  return LMP_OK;
}

int lmp_jit_launch(void* handle, uint32_t grid, uint32_t block, void** args) {
  if (!handle) return fail(LMP_ERR_INVALID, "lmp_jit_launch: null handle");
  if (grid == 0 || block == 0 || block > 1024)
    return fail(LMP_ERR_INVALID, "lmp_jit_launch: bad launch shape");
  LMP_RUNTIME_OR_FAIL(rt);
  JitKernel* k = static_cast<JitKernel*>(handle);
  LMP_HIP_TRY(hipModuleLaunchKernel(k->fn, grid, 1, 1, block, 1, 1, 0,
                                    rt->stream, args, nullptr));
  return LMP_OK;
}

int lmp_jit_compiled_count(uint64_t* count) {
  if (!count) return fail(LMP_ERR_INVALID, "null count");
  JitCache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  *count = c.compiled;
  return LMP_OK;
}

}  // extern "C"
