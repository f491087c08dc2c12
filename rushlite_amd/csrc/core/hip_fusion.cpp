// Lazy-fusion backend of the HIP device (replaces NVRTCInductorBackend,
// nvrtc_backend.cpp:145-192, fused_graph.cpp:6-35, codegen.cpp:21-61).
//
// realize(root) grows one region backwards from the root through deferred
// elementwise nodes of one float type (float32, or float64 on the indexed
// path); every other input (already realised tensors, and
// non-fusible or too-distant pending nodes, which are realised first) becomes
// a leaf, deduplicated by identity so `a*a` loads `a` once.  Unlike the
// reference, operands of different shapes fuse: every leaf is indexed from
// the root's output index through its right-aligned broadcast strides, so
// `a*a + b` with b [M,1] and `exp(a)*b - relu(a)/(b+1)` each become a single
// kernel that reads a and b once and writes the result once.
//
// The region is keyed by a structural hash (op codes, wiring, clamp bounds,
// leaf broadcast layouts, output shape); a repeated graph costs a map lookup,
// with no source text built.  On a miss the region is turned into HIP source
// specialised to its shape: the layout is coalesced to the fewest dims, and
// when it reduces to rows x cols with each leaf contiguous or broadcast along
// the row, each lane of a one-shot grid produces one float4 (a workgroup owns
// a contiguous 4 KiB output tile) from 128-bit loads and stores it with a
// nontemporal hint; otherwise it decomposes the flat index with compile-time
// extents.  Kernels launch on the library stream without a
// device synchronisation (the reference synchronises every launch,
// nvrtc_backend.cpp:135-141).
#include <cstring>
#include <mutex>
#include <sstream>
#include <unordered_map>
#include <unordered_set>

#include "ops.hpp"

namespace lmp::tensor::hip {
namespace {

constexpr size_t kMaxNodes = 96;
constexpr size_t kMaxLeaves = 16;
constexpr int kBlock = 256;

struct Region {
  std::vector<TensorImpl*> leaves;
  std::vector<TensorImpl*> nodes;  // topological, root last
  std::unordered_map<TensorImpl*, int> leaf_of;
  std::unordered_map<TensorImpl*, int> node_of;
  std::unordered_map<TensorImpl*, long> owners;  // shared_ptr owners of each input
};

// Regions are homogeneous float32 or float64: a node fuses when it and all
// of its inputs have one of those types and the same one.
bool fusible_node(const TensorImpl* t) {
  if (!t->is_deferred()) return false;
  const DataType dt = t->type();
  if (dt != DataType::Float32 && dt != DataType::Float64) return false;
  const auto& fn = t->lazy_op();
  if (!fn->is_fusible()) return false;
  for (const auto& in : fn->inputs)
    if (in->type() != dt) return false;
  return true;
}

void add_leaf(TensorImpl* t, Region& r) {
  if (r.leaf_of.count(t)) return;
  t->data();  // realise (may run the leaf's own fused region)
  r.leaf_of[t] = static_cast<int>(r.leaves.size());
  r.leaves.push_back(t);
}

void grow(TensorImpl* t, Region& r, bool is_root,
          const std::unordered_set<TensorImpl*>& forced) {
  if (r.node_of.count(t) || r.leaf_of.count(t)) return;
  if (!is_root && (!fusible_node(t) || forced.count(t) || r.nodes.size() >= kMaxNodes ||
                   r.leaves.size() >= kMaxLeaves)) {
    add_leaf(t, r);
    return;
  }
  for (const auto& in : t->lazy_op()->inputs) {
    r.owners[in.get()] = in.use_count();
    grow(in.get(), r, false, forced);
  }
  r.node_of[t] = static_cast<int>(r.nodes.size());
  r.nodes.push_back(t);
}

// Grow the region for `root`, then turn every interior node that something
// outside the region still owns (a variable, a saved input, another pending
// node) into a leaf, which realises it once as its own region; inlining it
// would compute it again whenever that other owner is realised.  Repeats
// until the region is closed.
Region build_region(TensorImpl* root) {
  std::unordered_set<TensorImpl*> forced;
  for (;;) {
    Region r;
    grow(root, r, true, forced);
    std::unordered_map<TensorImpl*, long> refs;
    for (TensorImpl* n : r.nodes)
      for (const auto& in : n->lazy_op()->inputs)
        if (r.node_of.count(in.get())) ++refs[in.get()];
    bool changed = false;
    for (TensorImpl* n : r.nodes) {
      if (n == root) continue;
      if (r.owners.at(n) > refs[n]) changed |= forced.insert(n).second;
    }
    if (!changed) return r;
  }
}

// ------------------------------------------------------------ layout

struct Group {
  int64_t extent;
  std::vector<int64_t> stride;  // per leaf
};

// Coalesce the output dims jointly over all leaves, innermost first.
std::vector<Group> coalesce(const std::vector<size_t>& shape,
                            const std::vector<std::vector<stride_t>>& strides) {
  std::vector<Group> g;
  const size_t nl = strides.size();
  for (size_t i = shape.size(); i-- > 0;) {
    const int64_t n = static_cast<int64_t>(shape[i]);
    if (n == 1) continue;
    if (!g.empty()) {
      Group& last = g.back();
      bool ok = true;
      for (size_t l = 0; l < nl && ok; ++l)
        ok = strides[l][i] == last.stride[l] * last.extent;
      if (ok) {
        last.extent *= n;
        continue;
      }
    }
    Group ng{n, std::vector<int64_t>(nl)};
    for (size_t l = 0; l < nl; ++l) ng.stride[l] = strides[l][i];
    g.push_back(std::move(ng));
  }
  return g;
}

struct Plan {
  bool vec = false;
  std::vector<Group> groups;
  uint64_t n = 0;      // output elements
  uint64_t nvec = 0;   // vec: output float4s
  int64_t cols4 = 0;   // vec: float4s per row
};

Plan make_plan(const Region& r, const std::vector<size_t>& shape, bool f64) {
  Plan p;
  p.n = shape_numel(shape);
  std::vector<std::vector<stride_t>> strides;
  for (TensorImpl* leaf : r.leaves) strides.push_back(padded_strides(leaf->shape(), shape.size()));
  p.groups = coalesce(shape, strides);
  // The float4 plan is float32 only; float64 regions use the indexed loop.
  if (f64 || p.groups.size() > 2 || p.n / 4 >= (1ull << 31)) return p;
  const int64_t cols = p.groups.empty() ? 1 : p.groups[0].extent;
  if (cols % 4 != 0) return p;
  for (size_t l = 0; l < r.leaves.size(); ++l) {
    const int64_t in = p.groups.empty() ? 0 : p.groups[0].stride[l];
    if (in != 0 && in != 1) return p;
    if (in == 1) {
      if ((reinterpret_cast<uintptr_t>(r.leaves[l]->raw()) & 15u) != 0) return p;
      if (p.groups.size() == 2 && p.groups[1].stride[l] % 4 != 0) return p;
    }
  }
  p.vec = true;
  p.cols4 = cols / 4;
  p.nvec = p.n / 4;
  return p;
}

// ---------------------------------------------------------- signature

uint64_t fnv1a(const std::vector<int64_t>& words) {
  uint64_t h = 1469598103934665603ull;
  for (int64_t w : words) {
    uint64_t v = static_cast<uint64_t>(w);
    for (int b = 0; b < 8; ++b) {
      h ^= (v >> (8 * b)) & 0xff;
      h *= 1099511628211ull;
    }
  }
  return h;
}

// A clamp bound as the kernel will see it: float bits, or double bits.
int64_t bound_bits(Scalar v, bool f64) {
  if (f64) {
    int64_t b;
    std::memcpy(&b, &v, sizeof b);
    return b;
  }
  const float f = static_cast<float>(v);
  uint32_t b;
  std::memcpy(&b, &f, sizeof b);
  return b;
}

std::vector<int64_t> signature(const Region& r, const std::vector<size_t>& shape,
                               const Plan& p, bool f64) {
  std::vector<int64_t> s;
  s.push_back(0x4c4d5046);  // tag
  s.push_back(f64 ? 8 : 4);
  s.push_back(static_cast<int64_t>(shape.size()));
  for (size_t d : shape) s.push_back(static_cast<int64_t>(d));
  s.push_back(static_cast<int64_t>(r.leaves.size()));
  for (TensorImpl* leaf : r.leaves) {
    s.push_back(static_cast<int64_t>(leaf->shape().size()));
    for (size_t d : leaf->shape()) s.push_back(static_cast<int64_t>(d));
  }
  s.push_back(p.vec ? 1 : 0);
  s.push_back(static_cast<int64_t>(r.nodes.size()));
  for (TensorImpl* n : r.nodes) {
    const auto& fn = n->lazy_op();
    s.push_back(static_cast<int64_t>(fn->kind()) * 256 + fn->code());
    if (fn->kind() == lazy::OpKind::Unary && fn->code() == LMP_UN_CLAMP) {
      s.push_back(bound_bits(fn->param0(), f64));
      s.push_back(bound_bits(fn->param1(), f64));
    }
    for (const auto& in : fn->inputs) {
      auto it = r.leaf_of.find(in.get());
      s.push_back(it != r.leaf_of.end() ? it->second : -1 - r.node_of.at(in.get()));
    }
  }
  return s;
}

// ------------------------------------------------------------- codegen

std::string substitute(std::string tmpl, const std::vector<std::string>& args) {
  for (size_t j = 0; j < args.size(); ++j) {
    const std::string ph = "{" + std::to_string(j) + "}";
    for (size_t pos = tmpl.find(ph); pos != std::string::npos;
         pos = tmpl.find(ph, pos + args[j].size()))
      tmpl.replace(pos, ph.size(), args[j]);
  }
  return tmpl;
}

// Emit the SSA chain for one lane value; `leaf(l)` spells leaf l's value.
template <typename LeafName>
void emit_chain(std::ostringstream& os, const Region& r, const std::string& indent,
                const std::string& dst, const char* type, LeafName leaf) {
  for (size_t m = 0; m < r.nodes.size(); ++m) {
    const auto& fn = r.nodes[m]->lazy_op();
    std::vector<std::string> args;
    for (const auto& in : fn->inputs) {
      auto it = r.leaf_of.find(in.get());
      args.push_back(it != r.leaf_of.end() ? leaf(it->second)
                                           : "t" + std::to_string(r.node_of.at(in.get())));
    }
    os << indent << "const " << type << " t" << m << " = " << substitute(fn->codegen_expr(), args)
       << ";\n";
  }
  os << indent << dst << " = t" << (r.nodes.size() - 1) << ";\n";
}

const char* kPrelude = R"(
typedef float lmp_v4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float lmp_clamp(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}
__device__ __forceinline__ double lmp_clamp(double x, double lo, double hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}
)";

std::string codegen(const Region& r, const Plan& p, const std::string& name, bool f64) {
  const char* T = f64 ? "double" : "float";
  std::ostringstream os;
  os << kPrelude;
  os << "extern \"C\" __global__ __launch_bounds__(" << kBlock << ") void " << name
     << "(" << T << "* __restrict__ out";
  for (size_t l = 0; l < r.leaves.size(); ++l)
    os << ", const " << T << "* __restrict__ in" << l;
  os << ") {\n";
  const size_t nl = r.leaves.size();
  if (p.vec) {
    // One-shot: workgroup b owns output float4s [256b, 256b + 256).
    const bool rows = p.groups.size() == 2;
    os << "  const unsigned v = blockIdx.x * " << kBlock << "u + threadIdx.x;\n";
    os << "  if (v >= " << p.nvec << "u) return;\n";
    if (rows) {
      os << "  const unsigned r = v / " << p.cols4 << "u;\n";
      os << "  const unsigned c = (v - r * " << p.cols4 << "u) * 4u;\n";
    } else {
      os << "  const unsigned r = 0u;\n  const unsigned c = v * 4u;\n";
    }
    for (size_t l = 0; l < nl; ++l) {
      const bool contig = !p.groups.empty() && p.groups[0].stride[l] == 1;
      const int64_t rs = rows ? p.groups[1].stride[l] : 0;
      if (contig)
        os << "  const lmp_v4 s" << l << " = *reinterpret_cast<const lmp_v4*>(in" << l
           << " + (unsigned long)r * " << rs << "ul + c);\n";
      else
        os << "  const float s" << l << " = in" << l << "[(unsigned long)r * " << rs
           << "ul];\n";
    }
    os << "  lmp_v4 o;\n";
    const char* comp[4] = {"x", "y", "z", "w"};
    for (int c = 0; c < 4; ++c) {
      os << "  {\n";
      emit_chain(os, r, "    ", std::string("o.") + comp[c], T, [&](int l) {
        const bool contig = !p.groups.empty() && p.groups[0].stride[l] == 1;
        return "s" + std::to_string(l) + (contig ? std::string(".") + comp[c] : "");
      });
      os << "  }\n";
    }
    os << "  __builtin_nontemporal_store(o, reinterpret_cast<lmp_v4*>(out) + v);\n}\n";
  } else {
    os << "  const unsigned long n = " << p.n << "ul;\n";
    os << "  for (unsigned long i = (unsigned long)blockIdx.x * " << kBlock
       << "u + threadIdx.x; i < n; i += (unsigned long)gridDim.x * " << kBlock << "u) {\n";
    os << "    unsigned long rest = i;\n";
    for (size_t l = 0; l < nl; ++l) os << "    unsigned long o" << l << " = 0;\n";
    for (size_t g = 0; g < p.groups.size(); ++g) {
      os << "    {\n      const unsigned long q = rest / " << p.groups[g].extent
         << "ul;\n      const unsigned long c = rest - q * " << p.groups[g].extent
         << "ul;\n      rest = q;\n";
      for (size_t l = 0; l < nl; ++l)
        if (p.groups[g].stride[l])
          os << "      o" << l << " += c * " << p.groups[g].stride[l] << "ul;\n";
      os << "    }\n";
    }
    os << "    " << T << " res;\n    {\n";
    emit_chain(os, r, "      ", "res", T, [&](int l) {
      return "in" + std::to_string(l) + "[o" + std::to_string(l) + "]";
    });
    os << "    }\n    out[i] = res;\n  }\n}\n";
  }
  return os.str();
}

// --------------------------------------------------------------- backend

struct Compiled {
  void* handle = nullptr;
  std::vector<int64_t> sig;
};

class HipFusionBackend : public lazy::LazyBackend {
 public:
  void realize(TensorImpl* root) override {
    if (!root->is_deferred()) return;
    if (!fusible_node(root)) {
      for (const auto& in : root->lazy_op()->inputs) in->data();
      root->lazy_op()->run_eager(*root);
      return;
    }
    const Region r = build_region(root);
    const bool f64 = root->type() == DataType::Float64;
    const std::vector<size_t> shape = root->shape();
    const size_t n = shape_numel(shape);
    Storage out(n * dtype_size(root->type()), DeviceType::HIP);
    if (n == 0) {
      root->set_realized(out);
      return;
    }
    const Plan p = make_plan(r, shape, f64);
    std::vector<int64_t> sig = signature(r, shape, p, f64);
    const uint64_t key = fnv1a(sig);
    void* handle = lookup(key, sig);
    if (!handle) {
      const std::string name = "lmp_fused";
      const std::string src = codegen(r, p, name, f64);
      hip_ok(lmp_jit_compile(key, src.c_str(), name.c_str(), &handle), "lmp_jit_compile");
      std::lock_guard<std::mutex> lock(mu_);
      cache_[key] = Compiled{handle, std::move(sig)};
      ++backend_stats().jit_compiles;
    } else {
      ++backend_stats().jit_cache_hits;
    }
    // Launch: one lane per float4 (vec, one-shot) or per element (grid-stride
    // loop, one-shot up to 2^30 workgroups).
    const uint64_t work = p.vec ? p.nvec : p.n;
    uint64_t grid = (work + kBlock - 1) / kBlock;
    grid = std::max<uint64_t>(1, std::min<uint64_t>(grid, uint64_t(1) << 30));
    std::vector<void*> ptrs;
    ptrs.reserve(r.leaves.size() + 1);
    ptrs.push_back(out.data());
    for (TensorImpl* leaf : r.leaves) ptrs.push_back(leaf->raw());
    std::vector<void*> args(ptrs.size());
    for (size_t i = 0; i < ptrs.size(); ++i) args[i] = &ptrs[i];
    hip_ok(lmp_jit_launch(handle, static_cast<uint32_t>(grid), kBlock, args.data()),
           "lmp_jit_launch");
    ++backend_stats().fused_launches;
    backend_stats().fused_nodes += r.nodes.size();
    root->set_realized(out);
  }

 private:
  void* lookup(uint64_t key, const std::vector<int64_t>& sig) {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = cache_.find(key);
    if (it == cache_.end()) return nullptr;
    LMP_CHECK(it->second.sig == sig) << "fusion cache: 64-bit graph hash collision";
    return it->second.handle;
  }
  std::mutex mu_;
  std::unordered_map<uint64_t, Compiled> cache_;
};

const bool kRegistered = [] {
  static HipFusionBackend instance;
  lazy::register_backend(DeviceType::HIP, &instance);
  return true;
}();

}  // namespace

// Source of the kernel a region would compile to; for tests and inspection.
std::string fused_source_for(TensorImpl* root) {
  LMP_CHECK(root->is_deferred()) << "tensor has no pending graph";
  const Region r = build_region(root);
  const bool f64 = root->type() == DataType::Float64;
  return codegen(r, make_plan(r, root->shape(), f64), "lmp_fused", f64);
}

}  // namespace lmp::tensor::hip
