// Native op frontend, broadcast metadata and the lazy-capture layer.
//
// Each elementwise frontend checks the capture mode, then either records a
// LazyFunction node (deferred tensor) or calls its device stub
// (native/expand_ops.cpp:28-39, native/unary_ops.cpp:23-33).  Floating-point
// reductions over the last axis are captured too (the reference never
// captures reductions), so a softmax row becomes one kernel.  Other
// reductions, matmul, transpose, views and memory ops are never captured;
// reading their inputs realises any pending graph (tensor_impl.cpp:33-36).
#pragma once

#include <chrono>
#include <memory>
#include <string>
#include <vector>

#include "tensor.hpp"

namespace lmp::tensor {

// ------------------------------------------------------------- metadata

// Right-aligned broadcast of two shapes (align_utils.cpp:18-40).
std::vector<size_t> broadcast_shapes(const std::vector<size_t>& a,
                                     const std::vector<size_t>& b);
// Contiguous strides of `in` aligned to `nd` output dims, 0 on size-1 dims
// (cpu/offset_util.cpp:7-28).
std::vector<stride_t> padded_strides(const std::vector<size_t>& in, size_t nd);

struct OpMeta {  // infer_meta.cpp:10-44
  DataType dtype;
  std::vector<size_t> shape;
  size_t size;
  bool expand;
};
OpMeta infer_unary(const TensorImpl& a);
OpMeta infer_binary(const TensorImpl& a, const TensorImpl& b);
OpMeta infer_reduct(const TensorImpl& a, size_t axis);

// ------------------------------------------------------------ dispatch

namespace ops {

using binary_fn = TensorImpl (*)(const TensorImpl&, const TensorImpl&);
using unary_fn = TensorImpl (*)(const TensorImpl&);
using clamp_fn = TensorImpl (*)(const TensorImpl&, Scalar, Scalar);
using abs_backward_fn = TensorImpl (*)(const TensorImpl&, const TensorImpl&);
using clamp_backward_fn = TensorImpl (*)(const TensorImpl&, const TensorImpl&,
                                         Scalar, Scalar);
using reduct_fn = TensorImpl (*)(const TensorImpl&, size_t);
using matmul_fn = TensorImpl (*)(const TensorImpl&, const TensorImpl&);
using transpose_fn = TensorImpl (*)(const TensorImpl&);
// C = op(A) * op(B) with either operand transposed in place of a
// materialised transpose; the reference spells these transpose + matmul
// (functions/matrix_ops.cpp:15-20).
using matmul_t_fn = TensorImpl (*)(const TensorImpl&, const TensorImpl&, bool,
                                   bool);
// C += op(A) * op(B) in place: gradient accumulation fused into the GEMM
// epilogue instead of a product followed by add_inplace (same rounding: the
// epilogue adds the finished fp32 product to C once).
using matmul_acc_fn = void (*)(TensorImpl& c, const TensorImpl&, const TensorImpl&,
                               bool, bool);
// x @ w + b with the bias added in the GEMM epilogue; the reference spells it
// matmul then broadcast add (LinearImpl::forward, layers/linear.cpp:21-26),
// with the same rounding.  With `relu` the epilogue also applies ReLU,
// clamp(t, 0, DBL_MAX) (layers/activation.cpp:14), as the Linear -> ReLU pair
// of a Sequential would.  Called only for float32 operands, a 2-D x and w,
// and a bias of w's column count.
using linear_fn = TensorImpl (*)(const TensorImpl& x, const TensorImpl& w,
                                 const TensorImpl& b, bool relu);

// A Linear's weight and bias gradients in one launch: c (+)= op(a) op(b) and
// s (+)= the column sums of op(b) (c [m, n], s n values; accumulate when
// acc_c / acc_s).  Float32 2-D operands only.
using matmul_colsum_fn = void (*)(const TensorImpl& a, const TensorImpl& b, bool ta, bool tb,
                                  TensorImpl& c, bool acc_c, TensorImpl& s, bool acc_s);

// matmul_colsum with ReLU's backward applied to b first (b' = b where
// 0 < mask < max, else 0; mask stored like b): a Linear -> ReLU pair's weight
// and bias gradients from its output gradient and its ReLU output.  b is not
// transposed.
using matmul_colsum_masked_fn = void (*)(const TensorImpl& a, const TensorImpl& b,
                                         const TensorImpl& mask, bool ta, TensorImpl& c,
                                         bool acc_c, TensorImpl& s, bool acc_s);

// A Linear's three gradients from its output gradient g [batch, out], input
// x [batch, in] and weight w [in, out]: dx (+)= g w^T, dw (+)= x^T g and
// db (+)= the column sums of g (accumulate when acc_*).  Float32 2-D operands
// only.
using linear_backward_fn = void (*)(const TensorImpl& x, const TensorImpl& w,
                                    const TensorImpl& g, TensorImpl& dx, bool acc_dx,
                                    TensorImpl& dw, bool acc_dw, TensorImpl& db, bool acc_db);

#define LMP_FOR_BINARY_OPS(_) \
  _(add) _(sub) _(mul) _(div) _(pow) _(eq) _(ne) _(ge) _(le) _(gt) _(lt)
#define LMP_FOR_UNARY_OPS(_) _(neg) _(exp) _(log) _(sqrt) _(abs) _(sin) _(cos) _(tan)
#define LMP_FOR_REDUCT_OPS(_) _(sum) _(max) _(min) _(prod)

#define LMP_DECL_BINARY(name)                     \
  LMP_DECLARE_DISPATCH(binary_fn, name##_stub)    \
  Tensor name(const Tensor& a, const Tensor& b);
#define LMP_DECL_UNARY(name)                   \
  LMP_DECLARE_DISPATCH(unary_fn, name##_stub)  \
  Tensor name(const Tensor& a);
#define LMP_DECL_REDUCT(name)                  \
  LMP_DECLARE_DISPATCH(reduct_fn, name##_stub) \
  Tensor name(const Tensor& a, size_t axis);

LMP_FOR_BINARY_OPS(LMP_DECL_BINARY)
LMP_FOR_UNARY_OPS(LMP_DECL_UNARY)
LMP_FOR_REDUCT_OPS(LMP_DECL_REDUCT)
#undef LMP_DECL_BINARY
#undef LMP_DECL_UNARY
#undef LMP_DECL_REDUCT

LMP_DECLARE_DISPATCH(clamp_fn, clamp_stub)
LMP_DECLARE_DISPATCH(abs_backward_fn, abs_backward_stub)
LMP_DECLARE_DISPATCH(clamp_backward_fn, clamp_backward_stub)
LMP_DECLARE_DISPATCH(matmul_fn, matmul_stub)
LMP_DECLARE_DISPATCH(transpose_fn, transpose_stub)
LMP_DECLARE_DISPATCH(matmul_t_fn, matmul_t_stub)
LMP_DECLARE_DISPATCH(matmul_acc_fn, matmul_acc_stub)
LMP_DECLARE_DISPATCH(linear_fn, linear_stub)
LMP_DECLARE_DISPATCH(matmul_colsum_fn, matmul_colsum_stub)
LMP_DECLARE_DISPATCH(matmul_colsum_masked_fn, matmul_colsum_masked_stub)
LMP_DECLARE_DISPATCH(linear_backward_fn, linear_backward_stub)

Tensor clamp(const Tensor& a, Scalar lo, Scalar hi);
Tensor abs_backward(const Tensor& input, const Tensor& grad);
Tensor clamp_backward(const Tensor& input, const Tensor& grad, Scalar lo, Scalar hi);
Tensor matmul(const Tensor& a, const Tensor& b);
// op(a) @ op(b): trans_a uses a^T, trans_b uses b^T (2-D only).
Tensor matmul_t(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b);
// c += op(a) @ op(b) in place (shapes must match exactly).
void matmul_acc(Tensor& c, const Tensor& a, const Tensor& b, bool trans_a, bool trans_b);
// x @ w + b (Linear's forward), followed by ReLU when `relu`; one fused GEMM
// where the backend has one.
Tensor linear(const Tensor& x, const Tensor& w, const Tensor& b, bool relu = false);
// *c (+)= op(a) @ op(b) and *s (+)= its column sums of op(b); an undefined *c
// or *s is allocated and written.  Returns false (and does nothing) where the
// device has no such form or the dtypes are not float32.
bool matmul_colsum(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b, Tensor* c,
                   Tensor* s);
// The same with ReLU's backward mask applied to b (b untransposed; mask the
// ReLU output, b's shape): *c (+)= op(a) @ b' and *s (+)= column sums of b'.
bool matmul_colsum_masked(const Tensor& a, const Tensor& b, const Tensor& mask, bool trans_a,
                          Tensor* c, Tensor* s);
// A Linear's gradients: *dx (+)= g @ w^T, *dw (+)= x^T @ g and *db (+)= the
// column sums of g; an undefined output is allocated and written.  Returns
// false (and does nothing) where the device has no such form, the dtypes are
// not float32 or the batch is empty.
bool linear_backward(const Tensor& x, const Tensor& w, const Tensor& g, Tensor* dx, Tensor* dw,
                     Tensor* db);
Tensor transpose(const Tensor& a);
Tensor reshape(const Tensor& a, std::vector<size_t> shape);
Tensor squeeze(const Tensor& a, size_t dim);
Tensor expand_dims(const Tensor& a, size_t dim);
Tensor to(const Tensor& a, DeviceType device);
void add_inplace(Tensor& dst, const Tensor& src);

}  // namespace ops

// Tensor-level operators with scalar overloads; a scalar becomes a [1] tensor
// of the other operand's dtype and device (native/overloads.hpp:16-28).
Tensor scalar_like(const Tensor& t, Scalar s);
// Route scalars made during a device-graph capture into `keep` (nullptr ends it).
void set_graph_keep_alive(std::vector<Tensor>* keep);
#define LMP_TENSOR_OPERATOR(sym, fn)                                        \
  inline Tensor operator sym(const Tensor& a, const Tensor& b) { return ops::fn(a, b); } \
  inline Tensor operator sym(const Tensor& a, Scalar s) {                   \
    return ops::fn(a, scalar_like(a, s));                                   \
  }                                                                         \
  inline Tensor operator sym(Scalar s, const Tensor& a) {                   \
    return ops::fn(scalar_like(a, s), a);                                   \
  }
LMP_TENSOR_OPERATOR(+, add)
LMP_TENSOR_OPERATOR(-, sub)
LMP_TENSOR_OPERATOR(*, mul)
LMP_TENSOR_OPERATOR(/, div)
LMP_TENSOR_OPERATOR(==, eq)
LMP_TENSOR_OPERATOR(!=, ne)
LMP_TENSOR_OPERATOR(>=, ge)
LMP_TENSOR_OPERATOR(<=, le)
LMP_TENSOR_OPERATOR(>, gt)
LMP_TENSOR_OPERATOR(<, lt)
#undef LMP_TENSOR_OPERATOR
inline Tensor operator-(const Tensor& a) { return ops::neg(a); }

// ---------------------------------------------------------------- lazy

namespace lazy {

// Capture flag, thread-local (capture_mode.cpp:7-22).
bool is_capture_enabled();
void set_capture_enabled(bool enable);
bool should_capture(DeviceType device);
class CaptureGuard {
 public:
  explicit CaptureGuard(bool enable);
  ~CaptureGuard();

 private:
  bool prev_;
};

// Op kinds shared by the lazy nodes, the structural graph hash and the code
// generator; codes equal lmp_binary_op / lmp_unary_op / lmp_reduce_op.
// Reduce nodes are keep-dims reductions over the last axis, recorded under
// capture so a region can end in (or pass through) a row reduction.  Fill
// nodes are constants (full_like under capture, e.g. the ones of
// SummationBackward): no inputs, param0() is the value.
enum class OpKind : uint8_t { Binary, Unary, Reduce, Fill };

// A deferred elementwise node (lazy_function.hpp:11-22).  codegen_expr()
// returns the node's expression with {0}/{1} for its operands, in the HIP
// spelling that matches the eager kernels' functors bit for bit.
struct LazyFunction {
  std::vector<std::shared_ptr<TensorImpl>> inputs;
  explicit LazyFunction(std::vector<std::shared_ptr<TensorImpl>> ins)
      : inputs(std::move(ins)) {}
  virtual ~LazyFunction() = default;
  virtual std::shared_ptr<TensorImpl> infer_output() const = 0;
  virtual void run_eager(TensorImpl& out) = 0;
  virtual std::string codegen_expr() const = 0;
  virtual bool is_fusible() const = 0;
  virtual OpKind kind() const = 0;
  virtual int code() const = 0;  // lmp_binary_op or lmp_unary_op value
  virtual Scalar param0() const { return 0; }
  virtual Scalar param1() const { return 0; }
};

struct LazyBackend {  // lazy_backend.hpp:15-35
  virtual ~LazyBackend() = default;
  virtual void realize(TensorImpl* t) = 0;
  // Several pending tensors at once (e.g. an optimizer's parameter updates);
  // targets[i], when not null, is a buffer root i may be computed straight
  // into (as realize_into).  The default realises them one by one.
  virtual void realize_many(const std::vector<TensorImpl*>& roots,
                            const std::vector<const Storage*>& targets) {
    (void)targets;
    for (TensorImpl* t : roots)
      if (t->is_deferred()) realize(t);
  }
  // Realises pending `root` straight into `target` (a buffer of its size that
  // its own region reads at most at the output's index) and then shares it;
  // false when the backend cannot (root is then realised elsewhere).
  virtual bool realize_into(TensorImpl* root, const Storage& target) {
    (void)target;
    realize(root);
    return false;
  }
};
LazyBackend* backend(DeviceType dev);
void register_backend(DeviceType dev, LazyBackend* b);

std::shared_ptr<TensorImpl> record(std::shared_ptr<LazyFunction> fn);
void realize(TensorImpl* t);
// Realises every pending tensor of `roots` (all on one device) through its
// backend's realize_many; `targets` is empty or one entry (or null) per root.
void realize_many(const std::vector<TensorImpl*>& roots,
                  const std::vector<const Storage*>& targets);
// LazyBackend::realize_into of root's device.
bool realize_into(TensorImpl* root, const Storage& target);

// p0/p1 are clamp backward's bounds (LMP_BIN_CLAMP_BACKWARD).
std::shared_ptr<LazyFunction> make_binary(int code,
                                          std::shared_ptr<TensorImpl> a,
                                          std::shared_ptr<TensorImpl> b, Scalar p0 = 0,
                                          Scalar p1 = 0);
std::shared_ptr<LazyFunction> make_unary(int code, std::shared_ptr<TensorImpl> a,
                                         Scalar p0 = 0, Scalar p1 = 0);
// param0() of a reduce node is its axis.
std::shared_ptr<LazyFunction> make_reduce(int code, std::shared_ptr<TensorImpl> a,
                                          size_t axis);
// A float32 / float64 constant of `shape` on `device`.
std::shared_ptr<LazyFunction> make_fill(const std::vector<size_t>& shape, DeviceType device,
                                        DataType dtype, Scalar value);

}  // namespace lazy

// Backend counters (launches and JIT activity), exposed for tests/bench.
struct BackendStats {
  uint64_t eager_launches = 0;
  uint64_t fused_launches = 0;
  uint64_t fused_nodes = 0;
  uint64_t jit_compiles = 0;
  uint64_t jit_cache_hits = 0;
  // Host time spent issuing work (ns): fused regions (region build, kernel
  // lookup, launch; leaves realised inside count too) and GEMMs.
  uint64_t fused_host_ns = 0;
  uint64_t gemm_host_ns = 0;
};
BackendStats& backend_stats();

// Adds the lifetime of the scope to a host-time counter.
class HostTimer {
 public:
  explicit HostTimer(uint64_t* acc) : acc_(acc), t0_(std::chrono::steady_clock::now()) {}
  ~HostTimer() {
    if (acc_)
      *acc_ += static_cast<uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                         std::chrono::steady_clock::now() - t0_)
                                         .count());
  }
  HostTimer(const HostTimer&) = delete;
  HostTimer& operator=(const HostTimer&) = delete;

 private:
  uint64_t* acc_;
  std::chrono::steady_clock::time_point t0_;
};

}  // namespace lmp::tensor
