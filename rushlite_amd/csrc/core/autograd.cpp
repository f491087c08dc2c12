// Autograd engine and per-op backward formulas.
//
// Formulas are Lamp3's (autograd/functions/expand_ops.cpp:15-40,
// unary_ops.cpp:16-28, reduct_ops.cpp:11-16, matrix_ops.cpp:8-35,
// view_ops.cpp:12-24), including its choices that differ from other
// libraries: the max/min gradient flows to every position equal to the
// result, clamp's gradient uses strict bounds, and the root of backward()
// need not be a scalar (it is seeded with ones).  Linear's backward products
// dY*W^T and X^T*dY run as transposed-operand GEMMs instead of a transpose
// followed by a GEMM.
#include <limits>
#include "autograd.hpp"

#include <algorithm>
#include <random>
#include <unordered_set>

namespace lmp::autograd {

using tensor::detail::UnsafeTensorAccessor;
namespace tops = tensor::ops;

// ---------------------------------------------------------------- grad mode

namespace {
thread_local bool t_grad = true;
}
bool is_grad_enabled() { return t_grad; }
void set_grad_enabled(bool enable) { t_grad = enable; }
GradGuard::GradGuard(bool enable) : prev_(t_grad) { t_grad = enable; }
GradGuard::~GradGuard() { t_grad = prev_; }

// ----------------------------------------------------------------- Variable

Variable::Variable(const Tensor& data, bool requires_grad)
    : impl_(std::make_shared<VariableImpl>()) {
  impl_->data = data;
  impl_->requires_grad = requires_grad;
}

Variable Variable::op_result(const Tensor& data, bool requires_grad) {
  Variable v;
  v.impl_ = std::make_shared<VariableImpl>();
  v.impl_->data = data;
  v.impl_->requires_grad = requires_grad;
  return v;
}

const Tensor& Variable::grad() const {
  LMP_CHECK(impl_->requires_grad) << "Cannot access grad() if requires_grad = false";
  if (!impl_->grad.defined()) {
    impl_->grad = tensor::zeros_like(impl_->data);
    impl_->grad_pass = 0;  // made outside any backward pass
  }
  return impl_->grad;
}

void Variable::zero_grad() {
  LMP_CHECK(requires_grad()) << "Cannot access grad() if requires_grad = false";
  // variable.cpp:25-29 installs a fresh zero tensor; leaving the gradient
  // unset is observably the same (grad() materialises zeros, the next
  // accumulation writes 0 + g) and saves a fill per parameter per step.
  impl_->grad = Tensor();
  impl_->grad_fn = nullptr;
}

namespace {
// A pending constant (a fill node, float32 or float64): its value as the
// tensor holds it.
bool pending_fill(const Tensor& t, Scalar* value) {
  const auto& ti = tensor::detail::UnsafeTensorAccessor::getImpl(t);
  if (!ti->is_deferred() || ti->lazy_op()->kind() != tensor::lazy::OpKind::Fill) return false;
  const Scalar v = ti->lazy_op()->param0();
  *value = t.type() == DataType::Float32 ? Scalar(float(v)) : v;
  return true;
}

// Backward passes run on this thread (VariableImpl::grad_pass).
thread_local uint64_t t_backward_pass = 0;

// Per-(device, dtype) [1] zero used to start a deferred gradient as 0 + g.
const Tensor& zero_scalar(DeviceType dev, DataType dt) {
  static std::vector<Tensor> cache(static_cast<size_t>(DeviceType::Count) * 6);
  Tensor& z = cache[static_cast<size_t>(dev) * 6 + static_cast<size_t>(dt)];
  if (!z.defined()) z = Tensor(std::vector<Scalar>{0.0}, {1}, dev, dt);
  return z;
}
}  // namespace

void Variable::incr_grad(const Tensor& g) {
  LMP_CHECK(requires_grad()) << "Cannot access grad() if requires_grad = false";
  if (!impl_->grad.defined()) {
    LMP_INTERNAL_ASSERT(g.shape() == impl_->data.shape())
        << "There should be no broadcasting in incr_grad";
    impl_->grad_pass = t_backward_pass;
    Scalar v;
    if (pending_fill(g, &v)) {
      // 0 + a constant is that constant (with -0.0 -> +0.0): the gradient
      // stays a constant node, which later reductions can fold.
      impl_->grad = tensor::full_like(g, 0.0 + v);
      return;
    }
    impl_->grad = tops::add(zero_scalar(g.device(), g.type()), g);
    return;
  }
  LMP_INTERNAL_ASSERT(g.shape() == impl_->grad.shape())
      << "There should be no broadcasting in incr_grad";
  if (tensor::detail::UnsafeTensorAccessor::getImpl(impl_->grad)->is_deferred()) {
    Scalar a, b;
    if (g.type() == impl_->grad.type() && pending_fill(impl_->grad, &a) && pending_fill(g, &b)) {
      // Two constants add to a constant, rounded as the add kernel rounds;
      // the gradient tensor is updated in place, so a handle taken from
      // .grad sees the sum (as add_inplace would give it).
      const Scalar sum = g.type() == DataType::Float32 ? Scalar(float(a) + float(b)) : a + b;
      tensor::detail::UnsafeTensorAccessor::getImpl(impl_->grad)
          ->replace_pending_constant(tensor::lazy::make_fill(g.shape(), g.device(), g.type(), sum));
      return;
    }
    if (impl_->grad_pass == t_backward_pass) {
      // Started in this pass (every other gradient is realised before
      // backward() returns), so nothing outside the pass holds it: the sum
      // stays pending and fuses with the pending terms, in the same order as
      // the in-place add.
      impl_->grad = tops::add(impl_->grad, g);
      return;
    }
    // A constant left pending by an earlier pass, which a handle taken from
    // .grad may share: written to its own buffer now (same tensor), then the
    // term is added in place below, as add_inplace does (variable.cpp:30-35).
    impl_->grad.realize();
  }
  // A realised gradient receiving a pending term (the backward formulas run
  // captured): grad + g is one fused kernel computed straight into the
  // gradient's buffer, so the buffer keeps its identity and g is never
  // materialised.  Same values as realising g and adding it in place.
  const auto& gi = tensor::detail::UnsafeTensorAccessor::getImpl(g);
  if (gi->is_deferred() && g.type() == impl_->grad.type() &&
      tensor::lazy::backend(g.device()) != nullptr) {
    Tensor sum;
    {
      tensor::lazy::CaptureGuard capture(true);
      sum = tops::add(impl_->grad, g);
    }
    const auto& gradi = tensor::detail::UnsafeTensorAccessor::getImpl(impl_->grad);
    if (!tensor::lazy::realize_into(tensor::detail::UnsafeTensorAccessor::getImpl(sum).get(),
                                    gradi->storage()))
      impl_->grad.copy(sum);
    return;
  }
  tops::add_inplace(impl_->grad, g);  // variable.cpp:30-35
}

void Variable::incr_grad_matmul(const Tensor& a, const Tensor& b, bool trans_a,
                                bool trans_b) {
  LMP_CHECK(requires_grad()) << "Cannot access grad() if requires_grad = false";
  if (!impl_->grad.defined()) {
    // A GEMM accumulates from +0, so its product equals 0 + product exactly.
    impl_->grad = tops::matmul_t(a, b, trans_a, trans_b);
    impl_->grad_pass = t_backward_pass;
    LMP_INTERNAL_ASSERT(impl_->grad.shape() == impl_->data.shape())
        << "There should be no broadcasting in incr_grad";
    return;
  }
  tops::matmul_acc(impl_->grad, a, b, trans_a, trans_b);
}

bool Variable::incr_grad_linear(Variable& w, Variable& b, const Tensor& x, const Tensor& g,
                                const Tensor* relu_out, Variable* xv) {
  LMP_CHECK(w.requires_grad() && b.requires_grad())
      << "Cannot access grad() if requires_grad = false";
  const size_t n = g.shape().size() == 2 ? g.shape()[1] : 0;
  if (b.impl_->data.numel() != n || w.impl_->data.shape().size() != 2) return false;
  LMP_INTERNAL_ASSERT(!(xv && relu_out)) << "the input gradient is not formed with a mask";
  // An input that is also the weight or the bias accumulates through the
  // separate calls.
  if (xv && (xv->impl_ == w.impl_ || xv->impl_ == b.impl_)) return false;
  Tensor wg = w.impl_->grad, bg = b.impl_->grad, xg;
  // Accumulation is in place on realised buffers (their identity is kept).
  if (wg.defined()) wg.realize();
  if (bg.defined()) bg.realize();
  if (xv) {
    LMP_CHECK(xv->requires_grad()) << "Cannot access grad() if requires_grad = false";
    xg = xv->impl_->grad;
    if (xg.defined()) xg.realize();
  }
  const bool done = xv         ? tops::linear_backward(x, w.impl_->data, g, &xg, &wg, &bg)
                    : relu_out ? tops::matmul_colsum_masked(x, g, *relu_out, true, &wg, &bg)
                               : tops::matmul_colsum(x, g, true, false, &wg, &bg);
  if (!done) return false;
  if (xv && !xv->impl_->grad.defined()) {
    // g @ w^T accumulated from +0 equals 0 + the product exactly.
    LMP_INTERNAL_ASSERT(xg.shape() == xv->impl_->data.shape())
        << "There should be no broadcasting in incr_grad";
    xv->impl_->grad = xg;
    xv->impl_->grad_pass = t_backward_pass;
  }
  if (!w.impl_->grad.defined()) {
    // A GEMM accumulates from +0, so its product equals 0 + product exactly;
    // the column sums start from +0 as well.
    LMP_INTERNAL_ASSERT(wg.shape() == w.impl_->data.shape())
        << "There should be no broadcasting in incr_grad";
    w.impl_->grad = wg;
    w.impl_->grad_pass = t_backward_pass;
  }
  if (!b.impl_->grad.defined()) {
    b.impl_->grad = bg.shape() == b.impl_->data.shape() ? bg : bg.reshape(b.impl_->data.shape());
    b.impl_->grad_pass = t_backward_pass;
  }
  return true;
}

void Variable::set_grad_fn(std::shared_ptr<Function> fn) {
  LMP_CHECK(requires_grad()) << "Cannot access grad() if requires_grad = false";
  impl_->grad_fn = std::move(fn);
}

void Variable::copy(const Variable& other) { impl_->data.copy(other.data()); }
void Variable::fill(Scalar value) { impl_->data.fill(value); }
void Variable::realize() { impl_->data.realize(); }

void Variable::backward() {
  LMP_CHECK(requires_grad()) << "Must be declared with requires_grad";
  // Depth-first post-order over saved inputs, then reversed
  // (variable.cpp:57-80), iteratively so deep graphs cannot overflow.
  std::vector<Variable> topo;
  std::unordered_set<const VariableImpl*> seen;
  struct Frame {
    Variable v;
    size_t next;
  };
  std::vector<Frame> stack;
  seen.insert(id());
  stack.push_back({*this, 0});
  while (!stack.empty()) {
    Frame& f = stack.back();
    const auto& fn = f.v.impl_->grad_fn;
    if (fn && f.next < fn->saved_inputs->size()) {
      const Variable& child = (*fn->saved_inputs)[f.next++];
      if (seen.insert(child.id()).second) stack.push_back({child, 0});
      continue;
    }
    topo.push_back(f.v);
    stack.pop_back();
  }
  std::reverse(topo.begin(), topo.end());
  {
    // The gradient formulas are elementwise chains over tensors the pass
    // already holds, so they run captured: each formula, with the first
    // accumulation into a gradient (0 + g), becomes one fused kernel on a
    // device with a lazy backend.  Values are those of the eager formulas
    // (fused kernels equal eager ones bit for bit).
    tensor::lazy::CaptureGuard capture(true);
    ++t_backward_pass;
    impl_->grad = tensor::ones_like(impl_->data);
    impl_->grad_pass = t_backward_pass;
    for (Variable& node : topo)
      if (node.impl_->grad_fn) node.impl_->grad_fn->apply({node});
  }
  // No pending gradient outlives backward(): later in-place updates of the
  // tensors a pending gradient reads must not change it.  Deepest first: the
  // region of an input's gradient reaches back to the seed and stores the
  // gradients held on the way as extra outputs, so a chain of pending
  // gradients is one kernel rather than one per gradient.  A constant
  // gradient (a pending fill: the seed, or a gradient that is the seed
  // passed through additions) reads nothing, so it may stay pending until it
  // is read.
  Scalar v;
  for (auto it = topo.rbegin(); it != topo.rend(); ++it)
    if (it->impl_->grad.defined() && !pending_fill(it->impl_->grad, &v))
      it->impl_->grad.realize();
}

// ------------------------------------------------------------ op recording

namespace {

using Backward = std::function<void(const Variable& out, variable_list& ins)>;

struct LambdaFunction : Function {
  Backward fn;
  variable_list apply(const variable_list& g) override {
    LMP_INTERNAL_ASSERT(g.size() == 1) << "Output size mismatch.";
    fn(g[0], *saved_inputs);
    return {};
  }
};

Variable record(const Tensor& result, variable_list inputs, const char* name,
                Backward bw) {
  bool rg = false;
  if (is_grad_enabled())
    for (const Variable& v : inputs) rg = rg || v.requires_grad();
  Variable out = Variable::op_result(result, rg);
  if (rg) {
    auto f = std::make_shared<LambdaFunction>();
    f->name = name;
    f->saved_inputs = std::make_unique<variable_list>(std::move(inputs));
    f->fn = std::move(bw);
    out.set_grad_fn(std::move(f));
  }
  return out;
}

Tensor sba(const Tensor& g, const Variable& like) {
  return detail::sum_broadcast_axis(g, like.data().shape());
}

[[noreturn]] void no_grad_formula(const char* op) {
  throw std::runtime_error(std::string("backward of ") + op + " is not implemented");
}

}  // namespace

namespace detail {
Tensor sum_broadcast_axis(const Tensor& grad, const std::vector<size_t>& orig) {
  if (grad.shape() == orig) return grad;
  Tensor g = grad;
  while (g.shape().size() > orig.size()) g = tops::sum(g, 0).squeeze(0);
  for (size_t i = 0; i < orig.size(); ++i)
    if (orig[i] == 1) g = tops::sum(g, i);
  LMP_INTERNAL_ASSERT(g.shape() == orig)
      << "Shape not correct: " << g.shape() << ". Expected: " << orig;
  return g;
}
}  // namespace detail

Variable scalar_var(const Variable& like, Scalar s) {
  return Variable(tensor::scalar_like(like.data(), s));
}

namespace ops {

#define LMP_BW_ARGS const Variable &out, variable_list &in
#define SELF in[0]
#define OTHER in[1]
#define G out.grad()

Variable add(const Variable& a, const Variable& b) {
  return record(tops::add(a.data(), b.data()), {a, b}, "AddBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(sba(G, SELF));
    if (OTHER.requires_grad()) OTHER.incr_grad(sba(G, OTHER));
  });
}

Variable sub(const Variable& a, const Variable& b) {
  return record(tops::sub(a.data(), b.data()), {a, b}, "SubtractBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(sba(G, SELF));
    if (OTHER.requires_grad()) OTHER.incr_grad(sba(-G, OTHER));
  });
}

Variable mul(const Variable& a, const Variable& b) {
  return record(tops::mul(a.data(), b.data()), {a, b}, "MultiplyBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(sba(OTHER.data() * G, SELF));
    if (OTHER.requires_grad()) OTHER.incr_grad(sba(SELF.data() * G, OTHER));
  });
}

Variable div(const Variable& a, const Variable& b) {
  return record(tops::div(a.data(), b.data()), {a, b}, "DivideBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(sba(G / OTHER.data(), SELF));
    if (OTHER.requires_grad())
      OTHER.incr_grad(sba((-1.0) * (out.data() * G / OTHER.data()), OTHER));
  });
}

Variable pow(const Variable& a, const Variable& b) {
  return record(tops::pow(a.data(), b.data()), {a, b}, "PowerBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad())
      SELF.incr_grad(sba(G * OTHER.data() * tops::pow(SELF.data(), OTHER.data() - 1.0),
                         SELF));
    if (OTHER.requires_grad())
      OTHER.incr_grad(sba(G * out.data() * tops::log(SELF.data()), OTHER));
  });
}

#define LMP_AG_COMPARE(name, label)                                              \
  Variable name(const Variable& a, const Variable& b) {                          \
    return record(tops::name(a.data(), b.data()), {a, b}, label "Backward",      \
                  [](LMP_BW_ARGS) { no_grad_formula(label); });                  \
  }
LMP_AG_COMPARE(eq, "Equal")
LMP_AG_COMPARE(ne, "NotEqual")
LMP_AG_COMPARE(ge, "GreaterEqual")
LMP_AG_COMPARE(le, "LessEqual")
LMP_AG_COMPARE(gt, "Greater")
LMP_AG_COMPARE(lt, "Less")
#undef LMP_AG_COMPARE

#define LMP_AG_UNARY_DEF(name, label, formula)                                  \
  Variable name(const Variable& a) {                                           \
    return record(tops::name(a.data()), {a}, label, [](LMP_BW_ARGS) {          \
      if (SELF.requires_grad()) SELF.incr_grad(formula);                       \
    });                                                                        \
  }
LMP_AG_UNARY_DEF(neg, "NegationBackward", -G)
LMP_AG_UNARY_DEF(exp, "ExponentialBackward", out.data() * G)
LMP_AG_UNARY_DEF(log, "LogarithmBackward", G / SELF.data())
LMP_AG_UNARY_DEF(sqrt, "SquareRootBackward", G / (out.data() + out.data()))
LMP_AG_UNARY_DEF(abs, "AbsoluteValueBackward", tops::abs_backward(SELF.data(), G))
LMP_AG_UNARY_DEF(sin, "SineBackward", G * tops::cos(SELF.data()))
LMP_AG_UNARY_DEF(cos, "CosineBackward", (-tops::sin(SELF.data())) * G)
LMP_AG_UNARY_DEF(tan, "TangentBackward", G + (G * out.data() * out.data()))
#undef LMP_AG_UNARY_DEF

Variable clamp(const Variable& a, Scalar lo, Scalar hi) {
  return record(tops::clamp(a.data(), lo, hi), {a}, "ClampBackward",
                [lo, hi](LMP_BW_ARGS) {
                  if (SELF.requires_grad())
                    SELF.incr_grad(tops::clamp_backward(SELF.data(), G, lo, hi));
                });
}

Variable sum(const Variable& a, size_t axis) {
  return record(tops::sum(a.data(), axis), {a}, "SummationBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(tensor::ones_like(SELF.data()) * G);
  });
}

Variable max(const Variable& a, size_t axis) {
  return record(tops::max(a.data(), axis), {a}, "MaximumBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(G * tops::eq(SELF.data(), out.data()));
  });
}

Variable min(const Variable& a, size_t axis) {
  return record(tops::min(a.data(), axis), {a}, "MinimumBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(G * tops::eq(SELF.data(), out.data()));
  });
}

Variable prod(const Variable& a, size_t axis) {
  return record(tops::prod(a.data(), axis), {a}, "ProductBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(G * (out.data() / SELF.data()));
  });
}

Variable matmul(const Variable& a, const Variable& b) {
  return record(tops::matmul(a.data(), b.data()), {a, b}, "MatrixMultiplicationBackward",
                [](LMP_BW_ARGS) {
                  if (SELF.requires_grad()) SELF.incr_grad_matmul(G, OTHER.data(), false, true);
                  if (OTHER.requires_grad()) OTHER.incr_grad_matmul(SELF.data(), G, true, false);
                });
}

// x @ w + b as one node: the gradients of the reference's AddBackward (bias
// branch, functions/expand_ops.cpp:15-40) and MatrixMultiplicationBackward
// (functions/matrix_ops.cpp:8-35), in that order.
namespace {
// Gradients of y = x @ w + b for the output gradient g (LinearImpl's
// matmul + broadcast add, layers/linear.cpp:21-26): dx = g w^T, and dw = x^T g
// with db = the dim-0 sum of g in one launch where the backend has the form.
void linear_backward(const Tensor& g, variable_list& in) {
  // All three gradients in one call (one launch for small products).
  if (in[0].requires_grad() && in[1].requires_grad() && in[2].requires_grad() &&
      Variable::incr_grad_linear(in[1], in[2], in[0].data(), g, nullptr, &in[0]))
    return;
  if (in[0].requires_grad()) in[0].incr_grad_matmul(g, in[1].data(), false, true);
  if (in[1].requires_grad() && in[2].requires_grad() &&
      Variable::incr_grad_linear(in[1], in[2], in[0].data(), g))
    return;
  if (in[2].requires_grad()) in[2].incr_grad(sba(g, in[2]));
  if (in[1].requires_grad()) in[1].incr_grad_matmul(in[0].data(), g, true, false);
}
}  // namespace

Variable linear(const Variable& x, const Variable& w, const Variable& b) {
  return record(tops::linear(x.data(), w.data(), b.data()), {x, w, b}, "LinearBackward",
                [](LMP_BW_ARGS) { linear_backward(G, in); });
}

Variable linear_relu(const Variable& x, const Variable& w, const Variable& b) {
  const DataType dt = x.data().type();
  if (dt != DataType::Float32 && dt != DataType::Float64)
    return clamp(linear(x, w, b), 0.0, std::numeric_limits<double>::max());
  // One node for Linear followed by ReLU.  ReLU's backward masks the gradient
  // by its input t (ClampBackward: g where 0 < t < max, functions/
  // unary_ops.cpp:27); for clamp(t, 0, max) the output gives the same mask for
  // every t, including NaN, +-0 and +-inf, so the pre-activation is not kept.
  return record(tops::linear(x.data(), w.data(), b.data(), true), {x, w, b},
                "LinearReluBackward", [](LMP_BW_ARGS) {
                  const Tensor h = out.data();
                  // An input that needs no gradient (a first layer): only the
                  // weight and bias gradients remain, and the GEMM applies the
                  // mask as it loads G, so the masked gradient is never stored.
                  if (!in[0].requires_grad() && in[1].requires_grad() && in[2].requires_grad() &&
                      Variable::incr_grad_linear(in[1], in[2], in[0].data(), G, &h))
                    return;
                  linear_backward(tops::clamp_backward(h, G, 0.0,
                                                       std::numeric_limits<double>::max()),
                                  in);
                });
}

Variable transpose(const Variable& a) {
  return record(tops::transpose(a.data()), {a}, "TransposeBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(tops::transpose(G));
  });
}

Variable reshape(const Variable& a, const std::vector<size_t>& shape) {
  return record(tops::reshape(a.data(), shape), {a}, "ReshapeBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(G.reshape(SELF.data().shape()));
  });
}

Variable squeeze(const Variable& a, size_t axis) {
  return record(tops::squeeze(a.data(), axis), {a}, "SqueezeBackward",
                [axis](LMP_BW_ARGS) {
                  if (SELF.requires_grad()) SELF.incr_grad(G.expand_dims(axis));
                });
}

Variable expand_dims(const Variable& a, size_t axis) {
  return record(tops::expand_dims(a.data(), axis), {a}, "ExpandDimsBackward",
                [axis](LMP_BW_ARGS) {
                  if (SELF.requires_grad()) SELF.incr_grad(G.squeeze(axis));
                });
}

Variable to(const Variable& a, DeviceType device) {
  return record(tops::to(a.data(), device), {a}, "ToBackward", [](LMP_BW_ARGS) {
    if (SELF.requires_grad()) SELF.incr_grad(G.to(SELF.data().device()));
  });
}

#undef G
#undef SELF
#undef OTHER
#undef LMP_BW_ARGS

}  // namespace ops

// ------------------------------------------------------------- constructors

namespace {
std::mt19937_64& rng() {
  static std::mt19937_64 g{std::random_device{}()};
  return g;
}
Variable from_values(const std::vector<Scalar>& v, const std::vector<size_t>& shape,
                     bool rg, DeviceType dev, DataType dt) {
  return Variable(Tensor(v, shape, dev, dt), rg);
}
}  // namespace

void manual_seed(uint64_t seed) { rng().seed(seed); }

Variable zeros(const std::vector<size_t>& shape, bool rg, DeviceType dev, DataType dt) {
  Tensor t = tensor::empty(shape, dev, dt);
  t.fill(0.0);
  return Variable(t, rg);
}

Variable ones(const std::vector<size_t>& shape, bool rg, DeviceType dev, DataType dt) {
  Tensor t = tensor::empty(shape, dev, dt);
  t.fill(1.0);
  return Variable(t, rg);
}

Variable rand(const std::vector<size_t>& shape, bool rg, DeviceType dev, DataType dt) {
  std::vector<Scalar> v(tensor::shape_numel(shape));
  std::uniform_real_distribution<double> d(0.0, 1.0);
  for (Scalar& x : v) x = d(rng());
  return from_values(v, shape, rg, dev, dt);
}

Variable randn(Scalar mean, Scalar stddev, const std::vector<size_t>& shape, bool rg,
               DeviceType dev, DataType dt) {
  std::vector<Scalar> v(tensor::shape_numel(shape));
  std::normal_distribution<double> d(mean, stddev);
  for (Scalar& x : v) x = d(rng());
  return from_values(v, shape, rg, dev, dt);
}

}  // namespace lmp::autograd
