// Lazy-fusion backend of the HIP device (replaces NVRTCInductorBackend,
// nvrtc_backend.cpp:145-192, fused_graph.cpp:6-35, codegen.cpp:21-61).
//
// realize(root) grows one region backwards from the root through deferred
// elementwise nodes of one float type (float32, or float64 on the indexed
// path); every other input (already realised tensors, and
// non-fusible or too-distant pending nodes, which are realised first) becomes
// a leaf, deduplicated by identity so `a*a` loads `a` once.  Interior nodes
// that are also owned elsewhere (autograd keeps every forward value) are
// stored by the same kernel as extra outputs, so a softmax and its loss, with
// every value the backward pass reads, is one kernel instead of one per value.  Unlike the
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
// the row, each lane of a one-shot grid produces one float4 (a one-wave
// workgroup owns a contiguous 1 KiB output tile) from 128-bit loads and
// stores it, with the nontemporal hint for large outputs; otherwise it
// decomposes the flat index with compile-time extents.  Kernels launch on the library stream without a
// device synchronisation (the reference synchronises every launch,
// nvrtc_backend.cpp:135-141).
#include <cstdio>
#include <functional>
#include <cstdlib>
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
constexpr size_t kMaxOutputs = 16;  // interior nodes stored beside the root
// Threads per workgroup of every fused kernel: one wave.  One-wave
// workgroups spread a one-shot grid's tiles more finely over the CUs than
// 256-thread ones: config 1's c = a*a + b over [8192,8192] (256 MiB read and
// written per call, rotating inputs) 6.45-6.46 -> 6.67-6.69 TB/s on one
// MI355X, the other fused kernels unchanged.  A row kernel then runs one row
// per workgroup.
constexpr int kBlock = 64;

// LMP_FUSION_LOG=1 prints one line per fused region (and why nodes were cut
// out of it) to stderr, to see how a graph splits into kernels.
bool fusion_log() {
  static const bool on = [] {
    const char* v = std::getenv("LMP_FUSION_LOG");
    return v && *v && *v != '0';
  }();
  return on;
}

std::string shape_text(const std::vector<size_t>& sh) {
  std::string t = "[";
  for (size_t i = 0; i < sh.size(); ++i) t += (i ? "," : "") + std::to_string(sh[i]);
  return t + "]";
}

void log_cut(const TensorImpl* n, const char* why) {
  if (fusion_log())
    std::fprintf(stderr, "[lmp fusion]   cut %s node %s kind %d code %d\n", why,
                 shape_text(n->shape()).c_str(), static_cast<int>(n->lazy_op()->kind()),
                 n->lazy_op()->code());
}

struct Region {
  std::vector<TensorImpl*> leaves;
  std::vector<TensorImpl*> nodes;  // topological, root last
  std::unordered_map<TensorImpl*, int> leaf_of;
  std::unordered_map<TensorImpl*, int> node_of;
  std::unordered_map<TensorImpl*, long> owners;  // shared_ptr owners of each input
  // Interior nodes the kernel also stores (in node order), and their index.
  std::vector<TensorImpl*> outputs;
  std::unordered_map<TensorImpl*, int> out_of;
  // Keeps every node and leaf alive while the region exists: realising a
  // leaf, or storing an interior node, drops lazy edges that may have been the
  // only owners of nodes beneath.
  std::vector<std::shared_ptr<TensorImpl>> hold;
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

// Leaves are only recorded while a region grows; they are realised once the
// region is closed (realise_leaves).  Realising during growth could realise a
// node already placed in the region and free the nodes beneath it.
void add_leaf(TensorImpl* t, Region& r) {
  if (r.leaf_of.count(t)) return;
  r.leaf_of[t] = static_cast<int>(r.leaves.size());
  r.leaves.push_back(t);
}

// Realise the inputs of a closed region (each may run its own region).  A
// closed region's interior nodes have no owner outside it, so no leaf's graph
// can reach them.
void realise_leaves(const Region& r) {
  for (TensorImpl* leaf : r.leaves) leaf->data();
}

void grow(TensorImpl* t, Region& r, bool is_root,
          const std::unordered_set<TensorImpl*>& forced) {
  if (r.node_of.count(t) || r.leaf_of.count(t)) return;
  if (!is_root && (!fusible_node(t) || forced.count(t) || r.nodes.size() >= kMaxNodes ||
                   r.leaves.size() >= kMaxLeaves)) {
    if (fusible_node(t) && !forced.count(t) && !r.leaf_of.count(t)) log_cut(t, "size limit");
    add_leaf(t, r);
    return;
  }
  for (const auto& in : t->lazy_op()->inputs) {
    if (!r.owners.count(in.get())) {
      r.owners[in.get()] = in.use_count();  // before the region's own hold
      r.hold.push_back(in);
    }
    grow(in.get(), r, false, forced);
  }
  r.node_of[t] = static_cast<int>(r.nodes.size());
  r.nodes.push_back(t);
}

bool is_reduce(const TensorImpl* t) {
  return t->is_deferred() && t->lazy_op()->kind() == lazy::OpKind::Reduce;
}

// ------------------------------------------------------------ row regions
//
// A region holding reduce nodes runs as a row kernel: one wave per row of the
// reduced shape S = [..., N], each lane holding its share of the row in
// registers.  Every node is either full (a shape that broadcasts to S with
// last dim N) or a row value (one that broadcasts to S with last dim 1, e.g.
// a [1, 1] loss seed), computed for each row; a reduce node turns a full value
// of shape S into a row value of shape S1 (S with last dim 1) with
// exactly the order of the eager wave-per-row kernel (row_reduce_wave_f32 for
// float32 rows with N % 4 == 0, row_reduce_wave otherwise: four interleaved
// accumulators, their pairwise combination, then a wave butterfly), so a
// fused softmax equals the eager one bit for bit.  Rows of 2048 or more, which
// the eager path reduces with a workgroup per row, are not fused.
constexpr int64_t kRowMax = 2048;

struct RowPlan {
  bool ok = false;
  std::vector<size_t> S;
  int64_t R = 0, N = 0;
  bool vec_order = false;  // float32 and N % 4 == 0: elements come in float4s
  bool vec_load = false;   // every full leaf can be read with aligned float4s
  std::vector<bool> full;               // per leaf: varies along the row
  std::vector<int64_t> row_stride;      // per leaf, in elements
};

// `sh` broadcasts to `S` (right-aligned, each dim equal or 1).
bool bcast_to(const std::vector<size_t>& sh, const std::vector<size_t>& S) {
  if (sh.size() > S.size()) return false;
  for (size_t i = 0; i < sh.size(); ++i) {
    const size_t d = sh[sh.size() - 1 - i];
    if (d != 1 && d != S[S.size() - 1 - i]) return false;
  }
  return true;
}

size_t last_dim(const std::vector<size_t>& sh) { return sh.empty() ? 1 : sh.back(); }

// A row kernel can store a node when every row owns its own slot (S or S1)
// or the node is a single value (stored once, by row 0).
bool row_storable(const TensorImpl* n, const std::vector<size_t>& S) {
  std::vector<size_t> S1 = S;
  S1.back() = 1;
  return n->shape() == S || n->shape() == S1 || shape_numel(n->shape()) == 1;
}

RowPlan row_plan(const Region& r) {
  RowPlan p;
  const TensorImpl* first = nullptr;
  for (TensorImpl* n : r.nodes)
    if (is_reduce(n)) {
      first = n;
      break;
    }
  if (!first) return p;
  p.S = first->lazy_op()->inputs[0]->shape();
  const size_t nd = p.S.size();
  if (nd == 0) return p;
  p.N = static_cast<int64_t>(p.S.back());
  if (p.N < 2 || p.N >= kRowMax) return p;
  p.R = static_cast<int64_t>(shape_numel(p.S)) / p.N;
  if (p.R > (int64_t(1) << 31)) return p;  // one wave per row, one-shot grid
  std::vector<size_t> S1 = p.S;
  S1.back() = 1;
  for (TensorImpl* n : r.nodes) {
    if (!bcast_to(n->shape(), p.S)) return p;
    if (is_reduce(n)) {
      const auto& fn = n->lazy_op();
      if (fn->inputs[0]->shape() != p.S || n->shape() != S1 ||
          static_cast<size_t>(fn->param0()) != nd - 1)
        return p;
    }
  }
  const TensorImpl* root = r.nodes.back();
  if (root->shape() != p.S && root->shape() != S1) return p;
  const bool f32 = root->type() == DataType::Float32;
  p.vec_order = f32 && p.N % 4 == 0;
  p.vec_load = p.vec_order;
  for (TensorImpl* leaf : r.leaves) {
    const std::vector<stride_t> st = padded_strides(leaf->shape(), nd);
    const int64_t last = st[nd - 1];
    if (last != 0 && last != 1) return p;
    // The leading dims must address rows linearly: offset = row * stride.
    int64_t rs = 0, span = 1;
    bool found = false;
    for (size_t i = nd - 1; i-- > 0;) {
      if (p.S[i] == 1) continue;
      if (!found) {
        rs = st[i];
        found = true;
      } else if (st[i] != rs * span) {
        return p;
      }
      span *= static_cast<int64_t>(p.S[i]);
    }
    p.full.push_back(last == 1);
    p.row_stride.push_back(rs);
    if (last == 1 && (rs % 4 != 0 || (reinterpret_cast<uintptr_t>(leaf->raw()) & 15u) != 0))
      p.vec_load = false;
  }
  p.ok = true;
  return p;
}

// Grow the region for `root` and close it.  An interior node that something
// outside the region still owns (a variable, a saved input, another pending
// node) must exist on its own after the kernel; inlining it alone would
// compute it again whenever that other owner is realised.  It becomes a
// second output of the same kernel where every lane can store it at its own
// index (any node of a row kernel; a node of the root's shape otherwise), and
// a leaf elsewhere, which realises it first as its own region.  Interior
// reduce nodes that cannot share a row kernel with the rest are made leaves
// too.  Repeats until the region is closed.
Region build_region(TensorImpl* root) {
  std::unordered_set<TensorImpl*> forced;
  for (;;) {
    Region r;
    grow(root, r, true, forced);
    std::unordered_map<TensorImpl*, long> refs;
    for (TensorImpl* n : r.nodes)
      for (const auto& in : n->lazy_op()->inputs)
        if (r.node_of.count(in.get())) ++refs[in.get()];
    // A constant (fill node) that others hold is a literal here and stays
    // pending for them: nothing to store.
    std::vector<TensorImpl*> shared;
    for (TensorImpl* n : r.nodes)
      if (n != root && r.owners.at(n) > refs[n] && n->lazy_op()->kind() != lazy::OpKind::Fill)
        shared.push_back(n);
    bool has_reduce = false;
    for (TensorImpl* n : r.nodes) has_reduce |= is_reduce(n);
    const RowPlan rp = has_reduce ? row_plan(r) : RowPlan{};
    const bool rows = rp.ok;
    bool changed = false;
    const auto cut = [&](TensorImpl* n, const char* why) {
      if (forced.insert(n).second) {
        changed = true;
        log_cut(n, why);
      }
    };
    if (rows) {
      for (TensorImpl* n : shared)
        if (!row_storable(n, rp.S)) cut(n, "held, not storable by rows");
    } else {
      for (TensorImpl* n : shared)
        if (n->shape() != root->shape()) cut(n, "held, not the root's shape");
      if (!changed && has_reduce)
        for (TensorImpl* n : r.nodes)
          if (n != root && is_reduce(n)) cut(n, "reduce outside a row plan");
    }
    // Past the output limit the deepest held nodes become leaves: each of
    // them realises the part of the graph below it (again storing up to the
    // limit), so a long chain splits into a few regions, not one per node.
    for (size_t k = 0; k + kMaxOutputs < shared.size(); ++k) cut(shared[k], "held, output limit");
    if (changed) continue;
    r.outputs = std::move(shared);
    for (size_t k = 0; k < r.outputs.size(); ++k) r.out_of[r.outputs[k]] = static_cast<int>(k);
    return r;
  }
}

// Build the region for `root` and realise its leaves.  A leaf's own region
// can reach an interior node of this one that both share, and store it as
// one of its outputs; the region is then built again with that node as a
// leaf.
Region settle_region(TensorImpl* root) {
  for (;;) {
    Region r = build_region(root);
    realise_leaves(r);
    bool stale = false;
    for (TensorImpl* n : r.nodes) stale |= !n->is_deferred();
    if (!stale) return r;
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

// 64-bit hash of the signature, a word at a time (a multiply-rotate round
// per word and a final avalanche); a hit is confirmed against the stored
// signature, so the hash only has to spread keys well.
uint64_t sig_hash(const std::vector<int64_t>& words) {
  uint64_t h = 0x243f6a8885a308d3ull ^ words.size();
  for (int64_t w : words) {
    uint64_t v = static_cast<uint64_t>(w) * 0x9e3779b97f4a7c15ull;
    v ^= v >> 32;
    h = ((h ^ v) << 27 | (h ^ v) >> 37) * 0xbf58476d1ce4e5b9ull;
  }
  h ^= h >> 31;
  h *= 0x94d049bb133111ebull;
  return h ^ (h >> 29);
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
                               const Plan& p, bool f64, const RowPlan& rp) {
  std::vector<int64_t> s;
  s.push_back(0x4c4d5046);  // tag
  s.push_back(f64 ? 8 : 4);
  s.push_back(rp.ok ? (rp.vec_load ? 3 : 2) : 0);
  for (size_t d : rp.S) s.push_back(static_cast<int64_t>(d));
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
    s.push_back(static_cast<int64_t>(n->shape().size()));
    for (size_t d : n->shape()) s.push_back(static_cast<int64_t>(d));
    if ((fn->kind() == lazy::OpKind::Unary && fn->code() == LMP_UN_CLAMP) ||
        (fn->kind() == lazy::OpKind::Binary && fn->code() == LMP_BIN_CLAMP_BACKWARD)) {
      s.push_back(bound_bits(fn->param0(), f64));
      s.push_back(bound_bits(fn->param1(), f64));
    }
    if (fn->kind() == lazy::OpKind::Reduce) s.push_back(static_cast<int64_t>(fn->param0()));
    if (fn->kind() == lazy::OpKind::Fill) s.push_back(bound_bits(fn->param0(), f64));
    for (const auto& in : fn->inputs) {
      auto it = r.leaf_of.find(in.get());
      s.push_back(it != r.leaf_of.end() ? it->second : -1 - r.node_of.at(in.get()));
    }
  }
  s.push_back(static_cast<int64_t>(r.outputs.size()));
  for (TensorImpl* n : r.outputs) s.push_back(r.node_of.at(n));
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

#define LMP_WAVE_SWAP_SRC(...) #__VA_ARGS__
const char* kPrelude = R"(
typedef float lmp_v4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float lmp_clamp(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}
__device__ __forceinline__ double lmp_clamp(double x, double lo, double hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}
)"
// The eager reductions' lane exchanges, the same text.
#include "../hip/wave_swap.inc"
    "\n";
#undef LMP_WAVE_SWAP_SRC

// Parameter names of one region in a kernel: its root output, the prefix of
// its interior outputs (xo0, ..) and of its leaves (in0, ..).  A kernel that
// runs several regions gives each its own names.
struct Names {
  std::string out, xo, in;
};
const Names kSingle{"out", "xo", "in"};
Names region_names(size_t i) {
  const std::string t = std::to_string(i);
  return {"out_" + t, "xo_" + t + "_", "in_" + t + "_"};
}

// One region's parameters: the root's output, the interior outputs, the leaves.
void emit_region_params(std::ostringstream& os, const Region& r, const char* T,
                        const Names& nm, bool first) {
  os << (first ? "" : ", ") << T << "* __restrict__ " << nm.out;
  for (size_t k = 0; k < r.outputs.size(); ++k) os << ", " << T << "* __restrict__ " << nm.xo << k;
  for (size_t l = 0; l < r.leaves.size(); ++l)
    os << ", const " << T << "* __restrict__ " << nm.in << l;
}

void emit_params(std::ostringstream& os, const Region& r, const std::string& name,
                 const char* T) {
  os << "extern \"C\" __global__ __launch_bounds__(" << kBlock << ") void " << name << "(";
  emit_region_params(os, r, T, kSingle, true);
  os << ") {\n";
}

// Leaves at least this large are read with the nontemporal hint: a tensor
// as large as the 256 MB memory-side cache cannot stay in it between uses,
// and reads that do not allocate there leave it to other data (a cold
// 256 MiB read + write: 84.4 -> 81.5 us on MI355X).  Below that size a leaf
// may still be in the cache from the kernel that wrote it (a warm 256 MiB
// re-read: 64.7 us with ordinary loads, 78.5 us nontemporal), so it keeps
// ordinary loads.  Leaf shapes are part of the structural key, so the choice
// is fixed by it.
constexpr size_t kStreamBytes = size_t(256) << 20;
// Outputs of more than half the MALL are stored with the nontemporal hint,
// smaller ones with ordinary stores, so that the kernel reading them next can
// find them in the MALL (measured on MI355X: a producer and its consumer over
// 64 MiB operands 56.8 -> 46.5 us with ordinary stores; 192 MiB and up,
// nontemporal stores are faster).  The output shape is part of the
// structural key, so the choice is fixed by it.
constexpr size_t kStreamStoreBytes = size_t(128) << 20;

// The body of a float4 (vec) region: block `block` owns output float4s
// [kBlock * block, kBlock * block + kBlock) (one-shot).
void emit_vec_body(std::ostringstream& os, const Region& r, const Plan& p, const Names& nm,
                   const std::string& block, bool stream_stores = false) {
  const size_t nl = r.leaves.size();
  const bool rows = p.groups.size() == 2;
  os << "  {\n  const unsigned v = " << block << " * " << kBlock << "u + threadIdx.x;\n";
  os << "  if (v < " << p.nvec << "u) {\n";
  if (rows) {
    os << "  const unsigned r = v / " << p.cols4 << "u;\n";
    os << "  const unsigned c = (v - r * " << p.cols4 << "u) * 4u;\n";
  } else {
    os << "  const unsigned r = 0u;\n  const unsigned c = v * 4u;\n";
  }
  for (size_t l = 0; l < nl; ++l) {
    const bool contig = !p.groups.empty() && p.groups[0].stride[l] == 1;
    const int64_t rs = rows ? p.groups[1].stride[l] : 0;
    const bool stream = r.leaves[l]->nbytes() >= kStreamBytes;
    if (contig && stream)
      os << "  const lmp_v4 s" << l << " = __builtin_nontemporal_load(reinterpret_cast<const lmp_v4*>("
         << nm.in << l << " + (unsigned long)r * " << rs << "ul + c));\n";
    else if (contig)
      os << "  const lmp_v4 s" << l << " = *reinterpret_cast<const lmp_v4*>(" << nm.in << l
         << " + (unsigned long)r * " << rs << "ul + c);\n";
    else
      os << "  const float s" << l << " = " << nm.in << l << "[(unsigned long)r * " << rs
         << "ul];\n";
  }
  os << "  lmp_v4 o;\n";
  for (size_t k = 0; k < r.outputs.size(); ++k) os << "  lmp_v4 x" << k << ";\n";
  const char* comp[4] = {"x", "y", "z", "w"};
  for (int c = 0; c < 4; ++c) {
    os << "  {\n";
    emit_chain(os, r, "    ", std::string("o.") + comp[c], "float", [&](int l) {
      const bool contig = !p.groups.empty() && p.groups[0].stride[l] == 1;
      return "s" + std::to_string(l) + (contig ? std::string(".") + comp[c] : "");
    });
    for (size_t k = 0; k < r.outputs.size(); ++k)
      os << "    x" << k << "." << comp[c] << " = t" << r.node_of.at(r.outputs[k]) << ";\n";
    os << "  }\n";
  }
  // Every output of a float4 region has the root's shape.
  const bool stream_out = stream_stores || p.n * sizeof(float) > kStreamStoreBytes;
  const auto store = [&](const std::string& val, const std::string& dst) {
    if (stream_out)
      os << "  __builtin_nontemporal_store(" << val << ", reinterpret_cast<lmp_v4*>(" << dst
         << ") + v);\n";
    else
      os << "  reinterpret_cast<lmp_v4*>(" << dst << ")[v] = " << val << ";\n";
  };
  for (size_t k = 0; k < r.outputs.size(); ++k)
    store("x" + std::to_string(k), nm.xo + std::to_string(k));
  store("o", nm.out);
  os << "  }\n  }\n";
}

std::string codegen(const Region& r, const Plan& p, const std::string& name, bool f64) {
  const char* T = f64 ? "double" : "float";
  std::ostringstream os;
  os << kPrelude;
  emit_params(os, r, name, T);
  const size_t nl = r.leaves.size();
  if (p.vec) {
    emit_vec_body(os, r, p, kSingle, "blockIdx.x");
    os << "}\n";
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
    for (size_t k = 0; k < r.outputs.size(); ++k)
      os << "      xo" << k << "[i] = t" << r.node_of.at(r.outputs[k]) << ";\n";
    os << "    }\n    out[i] = res;\n  }\n}\n";
  }
  return os.str();
}

// The body of an indexed region run one-shot: block `block` owns elements
// [kBlock * block, kBlock * block + kBlock), each decomposed into leaf offsets with
// compile-time extents and strides.
void emit_indexed_body(std::ostringstream& os, const Region& r, const Plan& p, const char* T,
                       const Names& nm, const std::string& block) {
  const size_t nl = r.leaves.size();
  os << "  {\n  const unsigned long i = (unsigned long)" << block << " * " << kBlock
     << "u + threadIdx.x;\n";
  os << "  if (i < " << p.n << "ul) {\n";
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
    return nm.in + std::to_string(l) + "[o" + std::to_string(l) + "]";
  });
  for (size_t k = 0; k < r.outputs.size(); ++k)
    os << "      " << nm.xo << k << "[i] = t" << r.node_of.at(r.outputs[k]) << ";\n";
  os << "    }\n    " << nm.out << "[i] = res;\n  }\n  }\n";
}

// One kernel for several independent elementwise regions (realize_all):
// region i owns workgroups [off_i, off_i + blocks_i), float4 lanes for a vec
// plan, one element per lane otherwise.
std::string codegen_multi(const std::vector<const Region*>& rs, const std::vector<const Plan*>& ps,
                          const std::vector<bool>& f64, const std::vector<uint64_t>& blocks,
                          const std::string& name) {
  std::ostringstream os;
  os << kPrelude;
  os << "extern \"C\" __global__ __launch_bounds__(" << kBlock << ") void " << name << "(";
  for (size_t i = 0; i < rs.size(); ++i)
    emit_region_params(os, *rs[i], f64[i] ? "double" : "float", region_names(i), i == 0);
  os << ") {\n";
  // A group is an optimizer's parameter updates, read again only by the next
  // step: past the store threshold as a whole, its outputs take nontemporal
  // stores even where one region alone would not (37.66 M updated parameters
  // of config 4: 69.1 -> 67.4 us).
  uint64_t out_bytes = 0;
  for (size_t i = 0; i < rs.size(); ++i)
    out_bytes += ps[i]->n * (f64[i] ? sizeof(double) : sizeof(float)) * (1 + rs[i]->outputs.size());
  const bool stream_group = out_bytes > kStreamStoreBytes;
  uint64_t off = 0;
  for (size_t i = 0; i < rs.size(); ++i) {
    os << (i ? "  else " : "  ") << "if (blockIdx.x < " << off + blocks[i] << "u)\n";
    const std::string block = "(blockIdx.x - " + std::to_string(off) + "u)";
    if (ps[i]->vec) emit_vec_body(os, *rs[i], *ps[i], region_names(i), block, stream_group);
    else emit_indexed_body(os, *rs[i], *ps[i], f64[i] ? "double" : "float", region_names(i), block);
    off += blocks[i];
  }
  os << "}\n";
  return os.str();
}

// Row kernel for a region with reduce nodes (see RowPlan).
std::string codegen_rows(const Region& r, const RowPlan& rp, const std::string& name,
                         bool f64) {
  const char* T = f64 ? "double" : "float";
  const bool vo = rp.vec_order;
  const int64_t NN = vo ? rp.N / 4 : rp.N;      // units a lane steps over
  const int64_t TT = (NN + 63) / 64;            // units per lane
  const int64_t E = vo ? TT * 4 : TT;           // elements per lane
  const auto elem_col = [&](int64_t e) {        // column of element e, as code
    std::ostringstream c;
    if (vo) c << "4u * (lane + " << 64 * (e / 4) << "u) + " << e % 4 << "u";
    else c << "lane + " << 64 * e << "u";
    return c.str();
  };
  const auto ok_of = [&](int64_t e) { return "ok" + std::to_string(vo ? e / 4 : e); };
  std::vector<bool> node_full(r.nodes.size());
  for (size_t m = 0; m < r.nodes.size(); ++m)
    node_full[m] = !is_reduce(r.nodes[m]) && static_cast<int64_t>(last_dim(r.nodes[m]->shape())) == rp.N;

  std::ostringstream os;
  os << kPrelude;
  emit_params(os, r, name, T);
  os << "  const unsigned lane = threadIdx.x & 63u;\n";
  os << "  const unsigned long row = (unsigned long)blockIdx.x * " << kBlock / 64
     << "ul + (threadIdx.x >> 6);\n";
  os << "  if (row >= " << rp.R << "ul) return;\n";
  for (int64_t t = 0; t < TT; ++t)
    os << "  const bool ok" << t << " = lane + " << 64 * t << "u < " << NN << "u;\n";
  // Leaves.
  for (size_t l = 0; l < r.leaves.size(); ++l) {
    const std::string base = "in" + std::to_string(l) + " + row * " +
                             std::to_string(rp.row_stride[l]) + "ul";
    if (!rp.full[l]) {
      os << "  const " << T << " l" << l << " = *(" << base << ");\n";
      continue;
    }
    if (rp.vec_load) {
      for (int64_t t = 0; t < TT; ++t) {
        os << "  const lmp_v4 q" << l << "_" << t << " = ok" << t
           << " ? *reinterpret_cast<const lmp_v4*>(" << base << " + 4u * (lane + " << 64 * t
           << "u)) : lmp_v4{0.0f, 0.0f, 0.0f, 0.0f};\n";
        const char* comp[4] = {"x", "y", "z", "w"};
        for (int c = 0; c < 4; ++c)
          os << "  const " << T << " l" << l << "_" << 4 * t + c << " = q" << l << "_" << t
             << "." << comp[c] << ";\n";
      }
    } else {
      for (int64_t e = 0; e < E; ++e)
        os << "  const " << T << " l" << l << "_" << e << " = " << ok_of(e) << " ? (" << base
           << ")[" << elem_col(e) << "] : " << T << "(0);\n";
    }
  }
  const auto arg = [&](const std::shared_ptr<TensorImpl>& in, int64_t e) {
    auto lt = r.leaf_of.find(in.get());
    if (lt != r.leaf_of.end())
      return "l" + std::to_string(lt->second) +
             (rp.full[lt->second] && e >= 0 ? "_" + std::to_string(e) : "");
    const int k = r.node_of.at(in.get());
    return "v" + std::to_string(k) + (node_full[k] && e >= 0 ? "_" + std::to_string(e) : "");
  };
  for (size_t m = 0; m < r.nodes.size(); ++m) {
    const auto& fn = r.nodes[m]->lazy_op();
    if (!is_reduce(r.nodes[m])) {
      const int64_t count = node_full[m] ? E : 1;
      for (int64_t e = 0; e < count; ++e) {
        std::vector<std::string> args;
        for (const auto& in : fn->inputs) args.push_back(arg(in, node_full[m] ? e : -1));
        os << "  const " << T << " v" << m << (node_full[m] ? "_" + std::to_string(e) : "")
           << " = " << substitute(fn->codegen_expr(), args) << ";\n";
      }
      continue;
    }
    // Reduction in the eager kernels' order.
    const int op = fn->code();
    std::string id;
    if (op == LMP_RED_SUM) id = f64 ? "0.0" : "0.0f";
    else if (op == LMP_RED_PROD) id = f64 ? "1.0" : "1.0f";
    else if (op == LMP_RED_MAX) id = f64 ? "__longlong_as_double(0xffefffffffffffffll)"
                                         : "__uint_as_float(0xff7fffffu)";
    else id = f64 ? "__longlong_as_double(0x7fefffffffffffffll)" : "__uint_as_float(0x7f7fffffu)";
    const auto comb = [&](const std::string& acc, const std::string& x) {
      switch (op) {
        case LMP_RED_SUM: return "(" + acc + " + " + x + ")";
        case LMP_RED_PROD: return "(" + acc + " * " + x + ")";
        case LMP_RED_MAX: return "(" + acc + " < " + x + " ? " + x + " : " + acc + ")";
        default: return "(" + x + " < " + acc + " ? " + x + " : " + acc + ")";
      }
    };
    const std::string P = "r" + std::to_string(m) + "_";
    const int W = vo ? 4 : 1;  // components per accumulator
    const auto acc = [&](int i, int c) { return P + "a" + std::to_string(i) + "_" + std::to_string(c); };
    const auto src = [&](int64_t t, int c) { return arg(fn->inputs[0], vo ? 4 * t + c : t); };
    os << "  " << T << " v" << m << ";\n  {\n";
    for (int i = 0; i < 4; ++i)
      for (int c = 0; c < W; ++c) os << "    " << T << " " << acc(i, c) << " = " << id << ";\n";
    os << "    unsigned " << P << "gd = 0u;\n";
    for (int64_t g = 0; 4 * g + 3 < TT; ++g) {
      os << "    if (lane + " << 64 * (4 * g + 3) << "u < " << NN << "u) {\n";
      for (int i = 0; i < 4; ++i)
        for (int c = 0; c < W; ++c)
          os << "      " << acc(i, c) << " = " << comb(acc(i, c), src(4 * g + i, c)) << ";\n";
      os << "      " << P << "gd = " << g + 1 << "u;\n    }\n";
    }
    for (int64_t t = 0; t < TT; ++t) {
      os << "    if (" << t << "u >= 4u * " << P << "gd && ok" << t << ") {\n";
      for (int c = 0; c < W; ++c)
        os << "      " << acc(0, c) << " = " << comb(acc(0, c), src(t, c)) << ";\n";
      os << "    }\n";
    }
    std::vector<std::string> b;
    for (int c = 0; c < W; ++c)
      b.push_back(comb(comb(acc(0, c), acc(1, c)), comb(acc(2, c), acc(3, c))));
    os << "    " << T << " " << P << "v = ";
    if (vo) {
      os << T << "(0);\n";
      for (int c = 0; c < 4; ++c)
        os << "    const " << T << " " << P << "b" << c << " = " << b[c] << ";\n";
      os << "    " << P << "v = " << comb(comb(P + "b0", P + "b1"), comb(P + "b2", P + "b3"))
         << ";\n";
    } else {
      os << b[0] << ";\n";
    }
    for (int off = 1; off <= 32; off <<= 1)
      os << "    { const " << T << " o = lmp_swap<" << off << ">(" << P << "v); " << P
         << "v = " << comb(P + "v", "o") << "; }\n";
    // Every lane goes on with lane 0's result, the value the eager kernel
    // stores (the lanes can differ where max/min tie +0 and -0).
    os << "    v" << m << " = lmp_lane0(" << P << "v);\n  }\n";
  }
  os << "  // stores\n";
  const auto store = [&](size_t m, const std::string& ptr) {
    if (!node_full[m]) {
      if (shape_numel(r.nodes[m]->shape()) == 1 && rp.R > 1)
        os << "  if (lane == 0u && row == 0ul) " << ptr << "[0] = v" << m << ";\n";
      else
        os << "  if (lane == 0u) " << ptr << "[row] = v" << m << ";\n";
      return;
    }
    const std::string obase = ptr + " + row * " + std::to_string(rp.N) + "ul";
    if (vo) {
      for (int64_t t = 0; t < TT; ++t)
        os << "  if (ok" << t << ") *reinterpret_cast<lmp_v4*>(" << obase << " + 4u * (lane + "
           << 64 * t << "u)) = lmp_v4{v" << m << "_" << 4 * t << ", v" << m << "_"
           << 4 * t + 1 << ", v" << m << "_" << 4 * t + 2 << ", v" << m << "_"
           << 4 * t + 3 << "};\n";
    } else {
      for (int64_t e = 0; e < E; ++e)
        os << "  if (ok" << e << ") (" << obase << ")[" << elem_col(e) << "] = v" << m << "_"
           << e << ";\n";
    }
  };
  for (size_t k = 0; k < r.outputs.size(); ++k)
    store(static_cast<size_t>(r.node_of.at(r.outputs[k])), "xo" + std::to_string(k));
  store(r.nodes.size() - 1, "out");
  os << "}\n";
  return os.str();
}

// --------------------------------------------------------------- backend

struct Compiled {
  void* handle = nullptr;
  std::vector<int64_t> sig;
};

// Storage the next fused root should be computed into (realize_into); taken
// by the root's realize() before any leaf is realised.
thread_local const Storage* t_target = nullptr;

// A region ready to launch: settled (leaves realised), outputs allocated.
struct Job {
  TensorImpl* root = nullptr;
  Region r;
  RowPlan rp;
  Plan p;
  bool f64 = false;
  std::vector<size_t> shape;
  Storage out{0, DeviceType::HIP};  // empty until prepare() allocates or takes a target
  std::vector<Storage> extra;
  // One lane per float4 (vec, one-shot), per row wave, or per element
  // (grid-stride loop, one-shot up to 2^30 workgroups).
  uint64_t blocks() const {
    const uint64_t work = rp.ok ? uint64_t(rp.R) * 64 : p.vec ? p.nvec : p.n;
    const uint64_t grid = (work + kBlock - 1) / kBlock;
    return std::max<uint64_t>(1, std::min<uint64_t>(grid, uint64_t(1) << 30));
  }
  // Workgroups when run inside a group (one-shot for the indexed plan too).
  uint64_t group_blocks() const {
    const uint64_t work = p.vec ? p.nvec : p.n;
    return std::max<uint64_t>(1, (work + kBlock - 1) / kBlock);
  }
  void push_args(std::vector<void*>& ptrs) const {
    ptrs.push_back(out.data());
    for (const Storage& x : extra) ptrs.push_back(x.data());
    for (TensorImpl* leaf : r.leaves) ptrs.push_back(leaf->raw());
  }
  void finish() {
    for (size_t k = 0; k < r.outputs.size(); ++k) r.outputs[k]->set_realized(extra[k]);
    root->set_realized(out);
  }
};

void run_eager_root(TensorImpl* root) {
  for (const auto& in : root->lazy_op()->inputs) in->data();
  root->lazy_op()->run_eager(*root);
}

class HipFusionBackend : public lazy::LazyBackend {
 public:
  bool realize_into(TensorImpl* root, const Storage& target) override {
    if (!root->is_deferred()) return false;
    t_target = &target;
    realize(root);
    t_target = nullptr;
    return root->raw() == target.data();
  }

  void realize(TensorImpl* root) override {
    HostScope scope;
    const Storage* target = t_target;
    t_target = nullptr;
    Job job;
    if (prepare(root, target, job)) launch_single(job);
  }

  // Several roots at once: the elementwise regions among them (an optimizer's
  // per-parameter updates) run as one kernel when their regions are
  // disjoint; row kernels, or all of them when regions overlap, are realised
  // one by one.  targets[i], when not null, is root i's realize_into buffer.
  void realize_many(const std::vector<TensorImpl*>& roots,
                    const std::vector<const Storage*>& targets) override {
    HostScope scope;
    std::vector<Job> jobs;
    jobs.reserve(roots.size());
    std::vector<size_t> job_root;
    for (size_t i = 0; i < roots.size(); ++i) {
      Job job;
      if (prepare(roots[i], targets[i], job)) {
        jobs.push_back(std::move(job));
        job_root.push_back(i);
      }
    }
    // Groupable when every region's nodes are still pending, pairwise
    // disjoint (constants excepted: each region inlines them as literals),
    // and hold no other job's root.
    std::unordered_set<TensorImpl*> seen;
    bool ok = true;
    for (const Job& j : jobs) {
      for (TensorImpl* n : j.r.nodes) {
        ok &= n->is_deferred();
        if (ok && (n == j.root || n->lazy_op()->kind() != lazy::OpKind::Fill))
          ok &= seen.insert(n).second;
      }
    }
    if (!ok) {
      // Overlapping regions: realise each on its own, from scratch.
      jobs.clear();
      for (size_t i = 0; i < roots.size(); ++i) {
        if (!roots[i]->is_deferred()) continue;
        t_target = targets[i];
        realize_region_outer(roots[i]);
      }
      return;
    }
    std::vector<Job*> group;
    size_t params = 0;
    const auto flush = [&] {
      if (group.size() == 1) launch_single(*group[0]);
      else if (!group.empty()) launch_group(group);
      group.clear();
      params = 0;
    };
    for (Job& j : jobs) {
      const size_t np = 1 + j.r.outputs.size() + j.r.leaves.size();
      // Row kernels, and regions large enough to fill the chip on their own
      // (2^20 workgroups is far past that), launch alone.
      if (j.rp.ok || j.group_blocks() > (uint64_t(1) << 20)) {
        launch_single(j);
        continue;
      }
      if (group.size() == kMaxGroup || params + np > kMaxGroupParams) flush();
      group.push_back(&j);
      params += np;
    }
    flush();
  }

 private:
  static constexpr size_t kMaxGroup = 16;
  static constexpr size_t kMaxGroupParams = 96;

  // Host time of outermost realisations only (nested ones are inside).
  struct HostScope {
    static int& depth() {
      thread_local int d = 0;
      return d;
    }
    HostTimer timer;
    HostScope() : timer(++depth() == 1 ? &backend_stats().fused_host_ns : nullptr) {}
    ~HostScope() { --depth(); }
  };

  void realize_region_outer(TensorImpl* root) { realize(root); }

  // Settles root's region and allocates its outputs (true), or realises root
  // without a fused kernel (false): not pending, not fusible, constants only,
  // a reduction no row kernel takes, or an empty output.
  bool prepare(TensorImpl* root, const Storage* target, Job& job) {
    if (!root->is_deferred()) return false;
    if (!fusible_node(root)) {
      run_eager_root(root);
      return false;
    }
    job.root = root;
    job.r = settle_region(root);
    const Region& r = job.r;
    if (r.leaves.empty()) {
      if (fusion_log())
        std::fprintf(stderr, "[lmp fusion] eager constants root %s\n",
                     shape_text(root->shape()).c_str());
      // Constants only (a fill, or arithmetic on fills): eager.
      run_eager_root(root);
      return false;
    }
    job.f64 = root->type() == DataType::Float64;
    job.rp = row_plan(r);
    if (is_reduce(root) && !job.rp.ok) {
      if (fusion_log())
        std::fprintf(stderr, "[lmp fusion] eager reduce root %s\n",
                     shape_text(root->shape()).c_str());
      // A reduction no row kernel can take (long rows, other layouts): eager.
      run_eager_root(root);
      return false;
    }
    job.shape = root->shape();
    const size_t n = shape_numel(job.shape);
    // Writing into the target is safe when every leaf stored there is read at
    // the output's own index: same shape, elementwise region.
    bool in_place =
        target && target->byte_size() == n * dtype_size(root->type()) && !job.rp.ok;
    if (in_place) {
      for (TensorImpl* leaf : r.leaves)
        if (leaf->raw() == target->data() && leaf->shape() != job.shape) in_place = false;
    }
    job.out = in_place ? *target : Storage(n * dtype_size(root->type()), DeviceType::HIP);
    job.extra.reserve(r.outputs.size());
    for (TensorImpl* x : r.outputs)
      job.extra.emplace_back(shape_numel(x->shape()) * dtype_size(x->type()), DeviceType::HIP);
    if (n == 0) {
      job.finish();
      return false;
    }
    job.p = make_plan(r, job.shape, job.f64);
    return true;
  }

  void* compiled(std::vector<int64_t> sig, const std::function<std::string()>& source) {
    const uint64_t key = sig_hash(sig);
    void* handle = lookup(key, sig);
    if (!handle) {
      const std::string name = "lmp_fused";
      const std::string src = source();
      hip_ok(lmp_jit_compile(key, src.c_str(), name.c_str(), &handle), "lmp_jit_compile");
      std::lock_guard<std::mutex> lock(mu_);
      cache_[key] = Compiled{handle, std::move(sig)};
      ++backend_stats().jit_compiles;
    } else {
      ++backend_stats().jit_cache_hits;
    }
    return handle;
  }

  void launch(void* handle, uint64_t grid, std::vector<void*>& ptrs) {
    std::vector<void*> args(ptrs.size());
    for (size_t i = 0; i < ptrs.size(); ++i) args[i] = &ptrs[i];
    hip_ok(lmp_jit_launch(handle, static_cast<uint32_t>(grid), kBlock, args.data()),
           "lmp_jit_launch");
    ++backend_stats().fused_launches;
  }

  void launch_single(Job& job) {
    const Region& r = job.r;
    void* handle = compiled(signature(r, job.shape, job.p, job.f64, job.rp), [&] {
      return job.rp.ok ? codegen_rows(r, job.rp, "lmp_fused", job.f64)
                       : codegen(r, job.p, "lmp_fused", job.f64);
    });
    std::vector<void*> ptrs;
    ptrs.reserve(r.leaves.size() + r.outputs.size() + 1);
    job.push_args(ptrs);
    launch(handle, job.blocks(), ptrs);
    backend_stats().fused_nodes += r.nodes.size();
    if (fusion_log())
      std::fprintf(stderr, "[lmp fusion] %s root %s nodes %zu leaves %zu outputs %zu\n",
                   job.rp.ok ? "rows" : job.p.vec ? "vec" : "indexed",
                   shape_text(job.shape).c_str(), r.nodes.size(), r.leaves.size(),
                   r.outputs.size());
    job.finish();
  }

  void launch_group(const std::vector<Job*>& group) {
    std::vector<int64_t> sig{0x4c4d504d, static_cast<int64_t>(group.size())};
    std::vector<const Region*> rs;
    std::vector<const Plan*> ps;
    std::vector<bool> f64;
    std::vector<uint64_t> blocks;
    uint64_t grid = 0;
    size_t nodes = 0;
    for (const Job* j : group) {
      const std::vector<int64_t> one = signature(j->r, j->shape, j->p, j->f64, j->rp);
      sig.push_back(static_cast<int64_t>(one.size()));
      sig.insert(sig.end(), one.begin(), one.end());
      rs.push_back(&j->r);
      ps.push_back(&j->p);
      f64.push_back(j->f64);
      blocks.push_back(j->group_blocks());
      grid += j->group_blocks();
      nodes += j->r.nodes.size();
    }
    void* handle = compiled(std::move(sig),
                            [&] { return codegen_multi(rs, ps, f64, blocks, "lmp_fused"); });
    std::vector<void*> ptrs;
    for (const Job* j : group) j->push_args(ptrs);
    launch(handle, grid, ptrs);
    backend_stats().fused_nodes += nodes;
    if (fusion_log())
      std::fprintf(stderr, "[lmp fusion] group of %zu regions, %zu nodes\n", group.size(),
                   nodes);
    for (Job* j : group) j->finish();
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
bool realize_into(TensorImpl* root, const Storage& target) {
  if (!root->is_deferred()) return false;
  t_target = &target;
  root->data();
  t_target = nullptr;
  return root->raw() == target.data();
}

std::string fused_source_for(TensorImpl* root) {
  LMP_CHECK(root->is_deferred()) << "tensor has no pending graph";
  const Region r = settle_region(root);
  const bool f64 = root->type() == DataType::Float64;
  const RowPlan rp = row_plan(r);
  if (rp.ok) return codegen_rows(r, rp, "lmp_fused", f64);
  return codegen(r, make_plan(r, root->shape(), f64), "lmp_fused", f64);
}

// Source of the one kernel realize_all would run for these elementwise roots
// (each region's plan, one-shot workgroup ranges); for tests and inspection.
std::string fused_group_source_for(const std::vector<TensorImpl*>& roots) {
  std::vector<Region> rs;
  std::vector<Plan> ps;
  std::vector<bool> f64;
  std::vector<uint64_t> blocks;
  rs.reserve(roots.size());
  ps.reserve(roots.size());
  for (TensorImpl* root : roots) {
    LMP_CHECK(root->is_deferred()) << "tensor has no pending graph";
    rs.push_back(settle_region(root));
    f64.push_back(root->type() == DataType::Float64);
    ps.push_back(make_plan(rs.back(), root->shape(), f64.back()));
    LMP_CHECK(!row_plan(rs.back()).ok) << "row regions are not grouped";
    const uint64_t work = ps.back().vec ? ps.back().nvec : ps.back().n;
    blocks.push_back(std::max<uint64_t>(1, (work + kBlock - 1) / kBlock));
  }
  std::vector<const Region*> rp;
  std::vector<const Plan*> pp;
  for (size_t i = 0; i < rs.size(); ++i) {
    rp.push_back(&rs[i]);
    pp.push_back(&ps[i]);
  }
  return codegen_multi(rp, pp, f64, blocks, "lmp_fused");
}

}  // namespace lmp::tensor::hip
