// Reverse-mode autograd over the tensor ops (Lamp3: autograd/variable.hpp,
// function.hpp, forward_function.hpp, functions/*, utils/*, grad_mode.hpp).
#pragma once

#include <functional>
#include <memory>
#include <vector>

#include "ops.hpp"

namespace lmp::autograd {

using tensor::DataType;
using tensor::DeviceType;
using tensor::Scalar;
using tensor::Tensor;

class Variable;
struct Function;
using variable_list = std::vector<Variable>;

// Grad mode, thread-local (grad_mode.cpp:5-16).
bool is_grad_enabled();
void set_grad_enabled(bool enable);
class GradGuard {
 public:
  explicit GradGuard(bool enable);
  ~GradGuard();

 private:
  bool prev_;
};

struct VariableImpl {
  Tensor data;
  // The gradient, materialised on demand.  Lamp3 allocates a zero tensor
  // when a variable with requires_grad is made (variable.hpp:24-28); here the
  // first accumulation instead writes 0 + g into a fresh buffer (or the GEMM
  // product straight into it), equal bit for bit to zeros + g without the
  // fill pass, and reading .grad before any accumulation materialises the
  // zeros.  Once it exists the buffer stays put: later accumulations are in
  // place, so a pointer taken from .grad stays valid across backward passes.
  Tensor grad;
  // The backward pass (a per-thread count) in which grad was started: a
  // gradient still pending from an earlier pass is a constant that a handle
  // taken from .grad may share, so a later term is added in place.
  uint64_t grad_pass = 0;
  std::shared_ptr<Function> grad_fn;
  bool requires_grad = false;
};

class Variable {
 public:
  Variable() = default;
  explicit Variable(const Tensor& data, bool requires_grad = false);

  const Tensor& grad() const;
  const Tensor& data() const noexcept { return impl_->data; }
  std::weak_ptr<Function> grad_fn() const noexcept { return impl_->grad_fn; }
  const std::shared_ptr<Function>& grad_fn_ptr() const noexcept { return impl_->grad_fn; }
  bool requires_grad() const noexcept { return impl_->requires_grad; }
  bool defined() const noexcept { return impl_ != nullptr; }

  void zero_grad();
  void incr_grad(const Tensor& g);
  // grad += op(a) @ op(b), fused into the GEMM epilogue.
  void incr_grad_matmul(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b);
  // A Linear's weight and bias gradients together: w.grad += x^T @ g and
  // b.grad += the column sums of g, in one launch where the backend has the
  // form (false, nothing done, otherwise).  With relu_out (a Linear -> ReLU
  // pair's output), g is first masked by ReLU's backward (g where
  // 0 < relu_out < max, else 0) as the GEMM loads it.  With xv (the variable
  // whose data is x; not with relu_out), xv.grad += g @ w^T as well, all three
  // in one launch where the products are small.
  static bool incr_grad_linear(Variable& w, Variable& b, const Tensor& x, const Tensor& g,
                               const Tensor* relu_out = nullptr, Variable* xv = nullptr);
  void set_grad_fn(std::shared_ptr<Function> fn);
  void copy(const Variable& other);
  void fill(Scalar value);
  void realize();
  void backward();

  // Result of a recorded op: gradient buffer deferred (see VariableImpl).
  static Variable op_result(const Tensor& data, bool requires_grad);
  const VariableImpl* id() const noexcept { return impl_.get(); }

 private:
  std::shared_ptr<VariableImpl> impl_;
};

// Backward node (function.hpp:12-22).  saved_inputs holds the forward
// inputs; apply receives {output variable} and accumulates into the inputs.
struct Function : std::enable_shared_from_this<Function> {
  std::unique_ptr<variable_list> saved_inputs;
  const char* name = "Function";
  virtual ~Function() = default;
  virtual variable_list apply(const variable_list& grad_outputs) = 0;
  variable_list operator()(const variable_list& g) { return apply(g); }
};

namespace detail {
// Sum a broadcast gradient back to `orig_shape` (utils/grad_utils.cpp:10-36).
Tensor sum_broadcast_axis(const Tensor& grad, const std::vector<size_t>& orig_shape);
}  // namespace detail

namespace ops {
#define LMP_AG_BINARY(name) Variable name(const Variable& a, const Variable& b);
LMP_FOR_BINARY_OPS(LMP_AG_BINARY)
#undef LMP_AG_BINARY
#define LMP_AG_UNARY(name) Variable name(const Variable& a);
LMP_FOR_UNARY_OPS(LMP_AG_UNARY)
#undef LMP_AG_UNARY
#define LMP_AG_REDUCT(name) Variable name(const Variable& a, size_t axis);
LMP_FOR_REDUCT_OPS(LMP_AG_REDUCT)
#undef LMP_AG_REDUCT
Variable clamp(const Variable& a, Scalar lo, Scalar hi);
Variable matmul(const Variable& a, const Variable& b);
Variable linear(const Variable& x, const Variable& w, const Variable& b);
// relu(linear(x, w, b)) as one node (Sequential's Linear -> ReLU pairs).
Variable linear_relu(const Variable& x, const Variable& w, const Variable& b);
Variable transpose(const Variable& a);
Variable reshape(const Variable& a, const std::vector<size_t>& shape);
Variable squeeze(const Variable& a, size_t axis);
Variable expand_dims(const Variable& a, size_t axis);
Variable to(const Variable& a, DeviceType device);
}  // namespace ops

// Scalars become [1] tensors of the variable's dtype and device
// (autograd/functions/overloads.hpp:16-29).
Variable scalar_var(const Variable& like, Scalar s);
#define LMP_VAR_OPERATOR(sym, fn)                                               \
  inline Variable operator sym(const Variable& a, const Variable& b) { return ops::fn(a, b); } \
  inline Variable operator sym(const Variable& a, Scalar s) { return ops::fn(a, scalar_var(a, s)); } \
  inline Variable operator sym(Scalar s, const Variable& a) { return ops::fn(scalar_var(a, s), a); }
LMP_VAR_OPERATOR(+, add)
LMP_VAR_OPERATOR(-, sub)
LMP_VAR_OPERATOR(*, mul)
LMP_VAR_OPERATOR(/, div)
LMP_VAR_OPERATOR(==, eq)
LMP_VAR_OPERATOR(!=, ne)
LMP_VAR_OPERATOR(>=, ge)
LMP_VAR_OPERATOR(<=, le)
LMP_VAR_OPERATOR(>, gt)
LMP_VAR_OPERATOR(<, lt)
#undef LMP_VAR_OPERATOR
inline Variable operator-(const Variable& a) { return ops::neg(a); }

// Constructors (utils/constructor.hpp:19-109).  rand/randn draw on the host
// from a generator seeded by manual_seed (random_device until then) and
// upload; randn's second argument is the standard deviation, as
// std::normal_distribution takes it in the reference (constructor.cpp:53).
Variable zeros(const std::vector<size_t>& shape, bool requires_grad = false,
               DeviceType device = tensor::DEFAULT_DEVICE,
               DataType dtype = tensor::DEFAULT_DTYPE);
Variable ones(const std::vector<size_t>& shape, bool requires_grad = false,
              DeviceType device = tensor::DEFAULT_DEVICE,
              DataType dtype = tensor::DEFAULT_DTYPE);
Variable rand(const std::vector<size_t>& shape, bool requires_grad = false,
              DeviceType device = tensor::DEFAULT_DEVICE,
              DataType dtype = tensor::DEFAULT_DTYPE);
Variable randn(Scalar mean, Scalar stddev, const std::vector<size_t>& shape,
               bool requires_grad = false, DeviceType device = tensor::DEFAULT_DEVICE,
               DataType dtype = tensor::DEFAULT_DTYPE);
void manual_seed(uint64_t seed);

}  // namespace lmp::autograd
