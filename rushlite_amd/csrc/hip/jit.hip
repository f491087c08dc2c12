// hipRTC module cache for the lazy-fusion backend (replaces the NVRTC cache
// of nvrtc_backend.cpp:19-128).  The caller keys modules by a 64-bit hash of
// the captured graph's structure, so a repeated graph costs one map lookup
// and no source generation.  Sources compile for the running device's exact
// gcnArchName (gfx950 on MI355X) with -O3 and -ffp-contract=off: eager Lamp3
// rounds after every op, so a fused a*a+b must not become an FMA.
//
// Compiled code objects also persist on disk, so a new process reuses every
// kernel an earlier one compiled (a hipRTC compile costs ~0.1-0.3 s).  The
// directory is $LMP_HIP_JIT_CACHE if set (an empty value disables the disk
// cache), else $XDG_CACHE_HOME/rushlite_amd/hiprtc, else
// $HOME/.cache/rushlite_amd/hiprtc.  A file is named by a 64-bit hash of
// (source, device arch, compile options, hipRTC version) and holds that whole
// identity next to the code object, so a hash collision or a stale file is a
// miss, never a wrong kernel.  Files are written to a temporary name and
// renamed, so concurrent processes never read a partial file.  The disk cache
// is best effort: any I/O failure falls back to compiling.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <fstream>
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
  uint64_t disk_loaded = 0;
  std::string arch;
  bool dir_known = false;
  std::string dir;  // empty: no disk cache
};

// Compile options; packed fp32 VALU forms stay disabled, as for the
// precompiled kernels.
std::vector<std::string> compile_options(const std::string& arch) {
  return {"--offload-arch=" + arch, "-O3", "-ffp-contract=off", "-std=c++17",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
}

uint64_t fnv1a(const std::string& s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char ch : s) {
    h ^= ch;
    h *= 1099511628211ull;
  }
  return h;
}

// mkdir -p; returns false when the directory cannot be made.
bool make_dirs(const std::string& path) {
  std::string cur;
  size_t pos = 0;
  while (pos != std::string::npos) {
    pos = path.find('/', pos + 1);
    cur = path.substr(0, pos);
    if (cur.empty()) continue;
    if (mkdir(cur.c_str(), 0755) != 0 && errno != EEXIST) return false;
  }
  struct stat st;
  return stat(path.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

std::string cache_dir() {
  if (const char* env = std::getenv("LMP_HIP_JIT_CACHE")) return env;
  if (const char* xdg = std::getenv("XDG_CACHE_HOME"); xdg && *xdg)
    return std::string(xdg) + "/rushlite_amd/hiprtc";
  if (const char* home = std::getenv("HOME"); home && *home)
    return std::string(home) + "/.cache/rushlite_amd/hiprtc";
  return "";
}

// Everything the code object depends on: the source, the target, the
// options, and the compiler's release down to its patch level (hipRTC
// reports major.minor only; the HIP runtime and driver versions it ships with
// carry the patch, so a point release of ROCm misses the cache).
std::string jit_identity(const std::string& source, const std::string& arch) {
  int major = 0, minor = 0, runtime = 0, driver = 0;
  hiprtcVersion(&major, &minor);
  if (hipRuntimeGetVersion(&runtime) != hipSuccess) runtime = -1;
  if (hipDriverGetVersion(&driver) != hipSuccess) driver = -1;
  (void)hipGetLastError();
  std::string id = "lmp-jit-v2\n" + arch + "\nhiprtc " + std::to_string(major) + "." +
                   std::to_string(minor) + "\nhip runtime " + std::to_string(runtime) +
                   "\nhip driver " + std::to_string(driver) + "\n";
  for (const auto& o : compile_options(arch)) id += o + "\n";
  id += source;
  return id;
}

std::string cache_path(const JitCache& c, const std::string& identity) {
  char name[32];
  std::snprintf(name, sizeof name, "%016llx.hsaco",
                static_cast<unsigned long long>(fnv1a(identity)));
  return c.dir + "/" + name;
}

// File layout: u64 identity length, identity bytes, u64 code length, code.
bool disk_load(const JitCache& c, const std::string& identity, std::vector<char>* code) {
  if (c.dir.empty()) return false;
  std::ifstream f(cache_path(c, identity), std::ios::binary);
  if (!f) return false;
  uint64_t n = 0;
  if (!f.read(reinterpret_cast<char*>(&n), sizeof n) || n != identity.size()) return false;
  std::string stored(n, '\0');
  if (!f.read(stored.data(), std::streamsize(n)) || stored != identity) return false;
  uint64_t m = 0;
  if (!f.read(reinterpret_cast<char*>(&m), sizeof m) || m == 0 || m > (1ull << 30))
    return false;
  code->resize(m);
  return static_cast<bool>(f.read(code->data(), std::streamsize(m)));
}

void disk_store(const JitCache& c, const std::string& identity, const std::vector<char>& code) {
  if (c.dir.empty()) return;
  const std::string path = cache_path(c, identity);
  const std::string tmp = path + ".tmp." + std::to_string(getpid());
  {
    std::ofstream f(tmp, std::ios::binary | std::ios::trunc);
    if (!f) return;
    const uint64_t n = identity.size(), m = code.size();
    f.write(reinterpret_cast<const char*>(&n), sizeof n);
    f.write(identity.data(), std::streamsize(n));
    f.write(reinterpret_cast<const char*>(&m), sizeof m);
    f.write(code.data(), std::streamsize(m));
    if (!f) {
      f.close();
      std::remove(tmp.c_str());
      return;
    }
  }
  if (std::rename(tmp.c_str(), path.c_str()) != 0) std::remove(tmp.c_str());
}

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
  if (!c.dir_known) {
    c.dir = cache_dir();
    if (!c.dir.empty() && !make_dirs(c.dir)) c.dir.clear();
    c.dir_known = true;
  }

  const std::string identity = jit_identity(source, c.arch);
  std::vector<char> code;
  const bool from_disk = disk_load(c, identity, &code);
  if (!from_disk) {
    hiprtcProgram prog;
    hiprtcResult r = hiprtcCreateProgram(&prog, source, "lmp_fused.hip", 0,
                                         nullptr, nullptr);
    if (r != HIPRTC_SUCCESS)
      return fail(LMP_ERR_JIT, std::string("hiprtcCreateProgram: ") +
                                   hiprtcGetErrorString(r));
    const std::vector<std::string> opts = compile_options(c.arch);
    std::vector<const char*> argv;
    for (const auto& o : opts) argv.push_back(o.c_str());
    r = hiprtcCompileProgram(prog, int(argv.size()), argv.data());
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
    code.resize(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
  }

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
  if (from_disk) {
    ++c.disk_loaded;
  } else {
    ++c.compiled;
    disk_store(c, identity, code);
  }
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
  count_kernel_launch();
  return LMP_OK;
}

int lmp_jit_compiled_count(uint64_t* count) {
  if (!count) return fail(LMP_ERR_INVALID, "null count");
  JitCache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  *count = c.compiled;
  return LMP_OK;
}

int lmp_jit_disk_loaded_count(uint64_t* count) {
  if (!count) return fail(LMP_ERR_INVALID, "null count");
  JitCache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  *count = c.disk_loaded;
  return LMP_OK;
}

}  // extern "C"
