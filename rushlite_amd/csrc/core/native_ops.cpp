// Op frontends, the capture flag, lazy nodes, record and realize.
// Lamp3 counterparts: native/*.cpp, lazy/*.cpp, lazy/functions/*.cpp.
#include <array>
#include <cmath>
#include <cstring>
#include <iomanip>
#include <limits>
#include <sstream>

#include "ops.hpp"

namespace lmp::tensor {

BackendStats& backend_stats() {
  static BackendStats s;
  return s;
}

namespace ops {

#define LMP_DEF_STUB_BINARY(name) LMP_DEFINE_DISPATCH(binary_fn, name##_stub)
#define LMP_DEF_STUB_UNARY(name) LMP_DEFINE_DISPATCH(unary_fn, name##_stub)
#define LMP_DEF_STUB_REDUCT(name) LMP_DEFINE_DISPATCH(reduct_fn, name##_stub)
LMP_FOR_BINARY_OPS(LMP_DEF_STUB_BINARY)
LMP_FOR_UNARY_OPS(LMP_DEF_STUB_UNARY)
LMP_FOR_REDUCT_OPS(LMP_DEF_STUB_REDUCT)
LMP_DEFINE_DISPATCH(clamp_fn, clamp_stub)
LMP_DEFINE_DISPATCH(abs_backward_fn, abs_backward_stub)
LMP_DEFINE_DISPATCH(clamp_backward_fn, clamp_backward_stub)
LMP_DEFINE_DISPATCH(matmul_fn, matmul_stub)
LMP_DEFINE_DISPATCH(transpose_fn, transpose_stub)
LMP_DEFINE_DISPATCH(matmul_t_fn, matmul_t_stub)
LMP_DEFINE_DISPATCH(matmul_acc_fn, matmul_acc_stub)
LMP_DEFINE_DISPATCH(linear_fn, linear_stub)
LMP_DEFINE_DISPATCH(matmul_colsum_fn, matmul_colsum_stub)
LMP_DEFINE_DISPATCH(matmul_colsum_masked_fn, matmul_colsum_masked_stub)
LMP_DEFINE_DISPATCH(linear_backward_fn, linear_backward_stub)

namespace {
using Acc = detail::UnsafeTensorAccessor;

Tensor wrap(TensorImpl&& t) {
  return Acc::fromImpl(std::make_shared<TensorImpl>(std::move(t)));
}
}  // namespace

// Binary ops: record under capture, else run the device stub.
#define LMP_DEF_BINARY(name, CODE)                                           \
  Tensor name(const Tensor& a, const Tensor& b) {                            \
    LMP_CHECK(a.device() == b.device()) << "Tensors are on different devices"; \
    const auto& ai = Acc::getImpl(a);                                        \
    const auto& bi = Acc::getImpl(b);                                        \
    if (lazy::should_capture(a.device()))                                    \
      return Acc::fromImpl(lazy::record(lazy::make_binary(CODE, ai, bi)));   \
    return wrap(name##_stub()(a.device(), *ai, *bi));                        \
  }
LMP_DEF_BINARY(add, LMP_BIN_ADD)
LMP_DEF_BINARY(sub, LMP_BIN_SUB)
LMP_DEF_BINARY(mul, LMP_BIN_MUL)
LMP_DEF_BINARY(div, LMP_BIN_DIV)
LMP_DEF_BINARY(pow, LMP_BIN_POW)
LMP_DEF_BINARY(eq, LMP_BIN_EQ)
LMP_DEF_BINARY(ne, LMP_BIN_NE)
LMP_DEF_BINARY(ge, LMP_BIN_GE)
LMP_DEF_BINARY(le, LMP_BIN_LE)
LMP_DEF_BINARY(gt, LMP_BIN_GT)
LMP_DEF_BINARY(lt, LMP_BIN_LT)
#undef LMP_DEF_BINARY

#define LMP_DEF_UNARY(name, CODE)                                         \
  Tensor name(const Tensor& a) {                                          \
    const auto& ai = Acc::getImpl(a);                                     \
    if (lazy::should_capture(a.device()))                                 \
      return Acc::fromImpl(lazy::record(lazy::make_unary(CODE, ai)));     \
    return wrap(name##_stub()(a.device(), *ai));                          \
  }
LMP_DEF_UNARY(neg, LMP_UN_NEG)
LMP_DEF_UNARY(exp, LMP_UN_EXP)
LMP_DEF_UNARY(log, LMP_UN_LOG)
LMP_DEF_UNARY(sqrt, LMP_UN_SQRT)
LMP_DEF_UNARY(abs, LMP_UN_ABS)
LMP_DEF_UNARY(sin, LMP_UN_SIN)
LMP_DEF_UNARY(cos, LMP_UN_COS)
LMP_DEF_UNARY(tan, LMP_UN_TAN)
#undef LMP_DEF_UNARY

Tensor clamp(const Tensor& a, Scalar lo, Scalar hi) {
  const auto& ai = Acc::getImpl(a);
  if (lazy::should_capture(a.device()))
    return Acc::fromImpl(lazy::record(lazy::make_unary(LMP_UN_CLAMP, ai, lo, hi)));
  return wrap(clamp_stub()(a.device(), *ai, lo, hi));
}

Tensor abs_backward(const Tensor& input, const Tensor& grad) {
  LMP_CHECK(input.device() == grad.device())
      << "abs_backward requires tensors on the same device";
  LMP_CHECK(input.shape() == grad.shape())
      << "abs_backward requires tensors with identical shapes";
  LMP_CHECK(input.type() == grad.type())
      << "abs_backward requires tensors with identical dtypes";
  if (lazy::should_capture(input.device()))
    return Acc::fromImpl(lazy::record(lazy::make_binary(
        LMP_BIN_ABS_BACKWARD, Acc::getImpl(input), Acc::getImpl(grad))));
  return wrap(abs_backward_stub()(input.device(), *Acc::getImpl(input),
                                  *Acc::getImpl(grad)));
}

Tensor clamp_backward(const Tensor& input, const Tensor& grad, Scalar lo, Scalar hi) {
  LMP_CHECK(input.device() == grad.device())
      << "clamp_backward requires tensors on the same device";
  LMP_CHECK(input.shape() == grad.shape())
      << "clamp_backward requires tensors with identical shapes";
  LMP_CHECK(input.type() == grad.type())
      << "clamp_backward requires tensors with identical dtypes";
  if (lazy::should_capture(input.device()))
    return Acc::fromImpl(lazy::record(lazy::make_binary(
        LMP_BIN_CLAMP_BACKWARD, Acc::getImpl(input), Acc::getImpl(grad), lo, hi)));
  return wrap(clamp_backward_stub()(input.device(), *Acc::getImpl(input),
                                    *Acc::getImpl(grad), lo, hi));
}

namespace {
// Under capture, a float32/float64 reduction over the last axis is recorded
// so the fusion backend can build it into a row kernel.
bool capture_reduction(const Tensor& a, size_t axis) {
  if (!lazy::should_capture(a.device())) return false;
  const DataType t = a.type();
  return (t == DataType::Float32 || t == DataType::Float64) && a.shape().size() >= 1 &&
         axis + 1 == a.shape().size() && a.numel() > 0;
}
}  // namespace

namespace {
// A reduction of a pending constant (a fill node: backward's ones seed, a
// SummationBackward ones) needs no pass over memory when its result is the
// same in every summation order: max and min are the value combined once
// with the identity (cpu/kernels.hpp:155-174), and a sum
// of n copies of an integer-valued v with |v| * n <= 2^24 (float32) or 2^53
// (float64) has only exact partial sums (a +-0 fill sums to +0 from the +0
// identity).  The result is then a constant of the keep-dims shape: pending
// under capture, filled otherwise.  Returns false where that does not hold.
bool fold_constant_reduction(const Tensor& a, size_t axis, int code, Tensor* out) {
  const auto& ai = Acc::getImpl(a);
  if (!ai->is_deferred() || ai->lazy_op()->kind() != lazy::OpKind::Fill) return false;
  const DataType t = a.type();
  if (t != DataType::Float32 && t != DataType::Float64) return false;
  if (axis >= a.shape().size() || a.shape()[axis] == 0) return false;
  const double n = static_cast<double>(a.shape()[axis]);
  const double v = t == DataType::Float32 ? double(float(ai->lazy_op()->param0()))
                                          : double(ai->lazy_op()->param0());
  if (std::isnan(v)) return false;
  double r;
  const bool f32 = t == DataType::Float32;
  const double big = f32 ? double(std::numeric_limits<float>::max())
                         : std::numeric_limits<double>::max();
  if (code == LMP_RED_MAX) {
    r = -big < v ? v : -big;  // combine(lowest(), v): -inf folds to lowest()
  } else if (code == LMP_RED_MIN) {
    r = v < big ? v : big;  // combine(max(), v): +inf folds to max()
  } else if (code == LMP_RED_SUM) {
    const double lim = t == DataType::Float32 ? 16777216.0 : 9007199254740992.0;
    if (v != std::trunc(v) || std::fabs(v) * n > lim) return false;
    r = v == 0.0 ? 0.0 : v * n;
  } else {
    return false;
  }
  std::vector<size_t> shape = a.shape();
  shape[axis] = 1;
  if (lazy::should_capture(a.device())) {
    *out = Acc::fromImpl(lazy::record(lazy::make_fill(shape, a.device(), t, r)));
  } else {
    *out = empty(shape, a.device(), t);
    out->fill(r);
  }
  return true;
}
}  // namespace

#define LMP_DEF_REDUCT(name, CODE)                                              \
  Tensor name(const Tensor& a, size_t axis) {                                   \
    const auto& ai = Acc::getImpl(a);                                           \
    Tensor folded;                                                              \
    if (fold_constant_reduction(a, axis, CODE, &folded)) return folded;         \
    if (capture_reduction(a, axis))                                             \
      return Acc::fromImpl(lazy::record(lazy::make_reduce(CODE, ai, axis)));    \
    return wrap(name##_stub()(a.device(), *ai, axis));                          \
  }
LMP_DEF_REDUCT(sum, LMP_RED_SUM)
LMP_DEF_REDUCT(max, LMP_RED_MAX)
LMP_DEF_REDUCT(min, LMP_RED_MIN)
LMP_DEF_REDUCT(prod, LMP_RED_PROD)
#undef LMP_DEF_REDUCT

Tensor matmul(const Tensor& a, const Tensor& b) {
  LMP_CHECK(a.device() == b.device()) << "Tensors must be on the same device";
  return wrap(matmul_stub()(a.device(), *Acc::getImpl(a), *Acc::getImpl(b)));
}

Tensor matmul_t(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b) {
  LMP_CHECK(a.device() == b.device()) << "Tensors must be on the same device";
  if (!matmul_t_stub().has(a.device())) {
    // Backends without the fused form: materialise the transposes.
    return matmul(trans_a ? transpose(a) : a, trans_b ? transpose(b) : b);
  }
  return wrap(matmul_t_stub()(a.device(), *Acc::getImpl(a), *Acc::getImpl(b),
                              trans_a, trans_b));
}

void matmul_acc(Tensor& c, const Tensor& a, const Tensor& b, bool trans_a, bool trans_b) {
  LMP_CHECK(a.device() == b.device() && a.device() == c.device())
      << "Tensors must be on the same device";
  if (!matmul_acc_stub().has(c.device())) {
    add_inplace(c, matmul_t(a, b, trans_a, trans_b));
    return;
  }
  matmul_acc_stub()(c.device(), *Acc::getImpl(c), *Acc::getImpl(a), *Acc::getImpl(b),
                    trans_a, trans_b);
}

bool matmul_colsum(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b, Tensor* c,
                   Tensor* s) {
  const DeviceType dev = a.device();
  if (!matmul_colsum_stub().has(dev) || b.device() != dev) return false;
  const auto f32 = [](const Tensor& t) { return t.type() == DataType::Float32; };
  if (!f32(a) || !f32(b) || a.shape().size() != 2 || b.shape().size() != 2) return false;
  if (c->defined() && (!f32(*c) || c->device() != dev)) return false;
  if (s->defined() && (!f32(*s) || s->device() != dev)) return false;
  const size_t m = a.shape()[trans_a ? 1 : 0], n = b.shape()[trans_b ? 0 : 1];
  // An empty inner dimension (a batch of zero rows) takes the unfused path:
  // a zero product and the identity of an empty sum.
  if (a.shape()[trans_a ? 0 : 1] == 0) return false;
  const bool acc_c = c->defined(), acc_s = s->defined();
  if (!acc_c)
    *c = wrap(TensorImpl(Storage(m * n * sizeof(float), dev), {m, n}, DataType::Float32));
  if (!acc_s) *s = wrap(TensorImpl(Storage(n * sizeof(float), dev), {n}, DataType::Float32));
  matmul_colsum_stub()(dev, *Acc::getImpl(a), *Acc::getImpl(b), trans_a, trans_b,
                       *Acc::getImpl(*c), acc_c, *Acc::getImpl(*s), acc_s);
  return true;
}

bool matmul_colsum_masked(const Tensor& a, const Tensor& b, const Tensor& mask, bool trans_a,
                          Tensor* c, Tensor* s) {
  const DeviceType dev = a.device();
  if (!matmul_colsum_masked_stub().has(dev) || b.device() != dev || mask.device() != dev)
    return false;
  const auto f32 = [](const Tensor& t) { return t.type() == DataType::Float32; };
  if (!f32(a) || !f32(b) || !f32(mask) || a.shape().size() != 2 || b.shape().size() != 2 ||
      mask.shape() != b.shape())
    return false;
  if (c->defined() && (!f32(*c) || c->device() != dev)) return false;
  if (s->defined() && (!f32(*s) || s->device() != dev)) return false;
  const size_t m = a.shape()[trans_a ? 1 : 0], n = b.shape()[1];
  if (a.shape()[trans_a ? 0 : 1] == 0) return false;  // empty batch: the unfused path
  const bool acc_c = c->defined(), acc_s = s->defined();
  if (!acc_c)
    *c = wrap(TensorImpl(Storage(m * n * sizeof(float), dev), {m, n}, DataType::Float32));
  if (!acc_s) *s = wrap(TensorImpl(Storage(n * sizeof(float), dev), {n}, DataType::Float32));
  matmul_colsum_masked_stub()(dev, *Acc::getImpl(a), *Acc::getImpl(b), *Acc::getImpl(mask),
                              trans_a, *Acc::getImpl(*c), acc_c, *Acc::getImpl(*s), acc_s);
  return true;
}

bool linear_backward(const Tensor& x, const Tensor& w, const Tensor& g, Tensor* dx, Tensor* dw,
                     Tensor* db) {
  const DeviceType dev = g.device();
  if (!linear_backward_stub().has(dev) || x.device() != dev || w.device() != dev) return false;
  const auto f32 = [](const Tensor& t) { return t.type() == DataType::Float32; };
  if (!f32(x) || !f32(w) || !f32(g) || x.shape().size() != 2 || w.shape().size() != 2 ||
      g.shape().size() != 2)
    return false;
  const size_t batch = x.shape()[0], in = x.shape()[1], out = w.shape()[1];
  if (w.shape()[0] != in || g.shape()[0] != batch || g.shape()[1] != out) return false;
  // An empty batch or layer takes the unfused path (zero products, empty sums).
  if (batch == 0 || in == 0 || out == 0) return false;
  for (const Tensor* t : {dx, dw, db})
    if (t->defined() && (!f32(*t) || t->device() != dev)) return false;
  const bool acc_dx = dx->defined(), acc_dw = dw->defined(), acc_db = db->defined();
  if (!acc_dx)
    *dx = wrap(TensorImpl(Storage(batch * in * sizeof(float), dev), {batch, in},
                          DataType::Float32));
  if (!acc_dw)
    *dw = wrap(TensorImpl(Storage(in * out * sizeof(float), dev), {in, out}, DataType::Float32));
  if (!acc_db) *db = wrap(TensorImpl(Storage(out * sizeof(float), dev), {out}, DataType::Float32));
  linear_backward_stub()(dev, *Acc::getImpl(x), *Acc::getImpl(w), *Acc::getImpl(g),
                         *Acc::getImpl(*dx), acc_dx, *Acc::getImpl(*dw), acc_dw,
                         *Acc::getImpl(*db), acc_db);
  return true;
}

Tensor linear(const Tensor& x, const Tensor& w, const Tensor& b, bool relu) {
  LMP_CHECK(x.device() == w.device() && x.device() == b.device())
      << "Tensors must be on the same device";
  const bool fused = linear_stub().has(x.device()) && x.type() == DataType::Float32 &&
                     w.type() == DataType::Float32 && b.type() == DataType::Float32 &&
                     x.shape().size() == 2 && w.shape().size() == 2 &&
                     x.shape()[1] == w.shape()[0] &&
                     (b.shape() == std::vector<size_t>{w.shape()[1]} ||
                      b.shape() == std::vector<size_t>{1, w.shape()[1]});
  if (!fused) {
    Tensor y = add(matmul(x, w), b);
    return relu ? clamp(y, 0.0, std::numeric_limits<double>::max()) : y;
  }
  return wrap(linear_stub()(x.device(), *Acc::getImpl(x), *Acc::getImpl(w), *Acc::getImpl(b),
                            relu));
}

Tensor transpose(const Tensor& a) {
  return wrap(transpose_stub()(a.device(), *Acc::getImpl(a)));
}

Tensor reshape(const Tensor& a, std::vector<size_t> shape) {
  return wrap(Acc::getImpl(a)->reshape(std::move(shape)));
}
Tensor squeeze(const Tensor& a, size_t dim) { return wrap(Acc::getImpl(a)->squeeze(dim)); }
Tensor expand_dims(const Tensor& a, size_t dim) {
  return wrap(Acc::getImpl(a)->expand_dims(dim));
}

Tensor to(const Tensor& a, DeviceType device) {
  LMP_CHECK(a.device() != device)
      << "Device argument must be different from current device.";
  Tensor out = empty(a.shape(), device, a.type());
  if (a.numel()) {
    void* src = const_cast<Tensor&>(a).data();
    copy_stub()(a.device(), device, src, out.data(), a.numel(), a.type(), a.type());
  }
  return out;
}

void add_inplace(Tensor& dst, const Tensor& src) {
  LMP_CHECK(dst.device() == src.device())
      << "add_inplace requires tensors on the same device";
  LMP_CHECK(dst.shape() == src.shape())
      << "add_inplace requires tensors with identical shapes";
  LMP_CHECK(dst.type() == src.type())
      << "add_inplace requires tensors with identical dtypes";
  void* s = const_cast<Tensor&>(src).data();
  add_inplace_stub()(dst.device(), dst.data(), s, dst.numel(), dst.type());
}

}  // namespace ops

// --------------------------------------------------------------------- lazy

namespace lazy {

namespace {
thread_local bool t_capture = false;

std::array<LazyBackend*, static_cast<size_t>(DeviceType::Count)>& registry() {
  static std::array<LazyBackend*, static_cast<size_t>(DeviceType::Count)> r{};
  return r;
}

// A Scalar bound converted to the tensor's float type on the host, as the
// eager launch does, and spelled by its bit pattern so inf (from DBL_MAX) and
// -0.0 survive.
std::string float_literal(Scalar v, bool f64) {
  std::ostringstream os;
  if (f64) {
    uint64_t bits;
    std::memcpy(&bits, &v, sizeof bits);
    os << "__longlong_as_double(0x" << std::hex << bits << "ll)";
  } else {
    const float f = static_cast<float>(v);
    uint32_t bits;
    std::memcpy(&bits, &f, sizeof bits);
    os << "__uint_as_float(0x" << std::hex << bits << "u)";
  }
  return os.str();
}

// Fused regions are float32 or float64 throughout; the spellings below call
// the same device math functions the eager kernels call for that type.
bool is_f64(const std::vector<std::shared_ptr<TensorImpl>>& ins) {
  return ins[0]->type() == DataType::Float64;
}

// Also the two backward functors of abs and clamp (input, grad), whose
// shapes and dtypes the frontends require to be equal.
struct BinaryFn : LazyFunction {
  int op;
  Scalar lo, hi;  // clamp backward's bounds
  BinaryFn(int code, std::vector<std::shared_ptr<TensorImpl>> ins, Scalar p0, Scalar p1)
      : LazyFunction(std::move(ins)), op(code), lo(p0), hi(p1) {}
  std::shared_ptr<TensorImpl> infer_output() const override {
    OpMeta m = infer_binary(*inputs[0], *inputs[1]);
    return std::make_shared<TensorImpl>(Storage(0, inputs[0]->device()), m.shape,
                                        m.dtype);
  }
  // Broadcast-compatible operands fuse too (the reference fuses only
  // equal shapes, elementwise_binary.cpp:11-13).
  bool is_fusible() const override { return true; }
  OpKind kind() const override { return OpKind::Binary; }
  int code() const override { return op; }
  Scalar param0() const override { return lo; }
  Scalar param1() const override { return hi; }
  void run_eager(TensorImpl& out) override {
    using namespace ops;
    const DeviceType d = inputs[0]->device();
    TensorImpl r = [&]() -> TensorImpl {
      switch (op) {
        case LMP_BIN_ABS_BACKWARD: return abs_backward_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_CLAMP_BACKWARD:
          return clamp_backward_stub()(d, *inputs[0], *inputs[1], lo, hi);
        case LMP_BIN_ADD: return add_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_SUB: return sub_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_MUL: return mul_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_DIV: return div_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_POW: return pow_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_EQ: return eq_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_NE: return ne_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_GE: return ge_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_LE: return le_stub()(d, *inputs[0], *inputs[1]);
        case LMP_BIN_GT: return gt_stub()(d, *inputs[0], *inputs[1]);
        default: return lt_stub()(d, *inputs[0], *inputs[1]);
      }
    }();
    out.set_realized(r.storage());
  }
  std::string codegen_expr() const override {
    const bool d = is_f64(inputs);
    const std::string one = d ? "1.0" : "1.0f", zero = d ? "0.0" : "0.0f";
    const auto cmp = [&](const char* op_text) {
      return std::string("({0} ") + op_text + " {1} ? " + one + " : " + zero + ")";
    };
    switch (op) {
      case LMP_BIN_ADD: return "({0} + {1})";
      case LMP_BIN_SUB: return "({0} - {1})";
      case LMP_BIN_MUL: return "({0} * {1})";
      case LMP_BIN_DIV: return "({0} / {1})";
      case LMP_BIN_POW: return d ? "pow({0}, {1})" : "powf({0}, {1})";
      case LMP_BIN_EQ: return cmp("==");
      case LMP_BIN_NE: return cmp("!=");
      case LMP_BIN_GE: return cmp(">=");
      case LMP_BIN_LE: return cmp("<=");
      case LMP_BIN_GT: return cmp(">");
      case LMP_BIN_LT: return cmp("<");
      // The eager functors: sign(x) * g with 0 at x == 0 (and NaN), and g
      // strictly inside (lo, hi), 0 elsewhere (and at NaN).
      case LMP_BIN_ABS_BACKWARD:
        return "({0} > " + zero + " ? {1} : ({0} < " + zero + " ? (-{1}) : " + zero + "))";
      default:
        return "(({0} > " + float_literal(lo, d) + " && {0} < " + float_literal(hi, d) +
               ") ? {1} : " + zero + ")";
    }
  }
};

struct UnaryFn : LazyFunction {
  int op;
  Scalar lo, hi;
  UnaryFn(int code, std::vector<std::shared_ptr<TensorImpl>> ins, Scalar p0, Scalar p1)
      : LazyFunction(std::move(ins)), op(code), lo(p0), hi(p1) {}
  std::shared_ptr<TensorImpl> infer_output() const override {
    return std::make_shared<TensorImpl>(Storage(0, inputs[0]->device()),
                                        inputs[0]->shape(), inputs[0]->type());
  }
  bool is_fusible() const override { return true; }
  OpKind kind() const override { return OpKind::Unary; }
  int code() const override { return op; }
  Scalar param0() const override { return lo; }
  Scalar param1() const override { return hi; }
  void run_eager(TensorImpl& out) override {
    using namespace ops;
    const DeviceType d = inputs[0]->device();
    TensorImpl r = [&]() -> TensorImpl {
      switch (op) {
        case LMP_UN_NEG: return neg_stub()(d, *inputs[0]);
        case LMP_UN_EXP: return exp_stub()(d, *inputs[0]);
        case LMP_UN_LOG: return log_stub()(d, *inputs[0]);
        case LMP_UN_SQRT: return sqrt_stub()(d, *inputs[0]);
        case LMP_UN_ABS: return abs_stub()(d, *inputs[0]);
        case LMP_UN_SIN: return sin_stub()(d, *inputs[0]);
        case LMP_UN_COS: return cos_stub()(d, *inputs[0]);
        case LMP_UN_TAN: return tan_stub()(d, *inputs[0]);
        default: return clamp_stub()(d, *inputs[0], lo, hi);
      }
    }();
    out.set_realized(r.storage());
  }
  // Same functions as the eager kernels.  abs is fabsf (the eager CPU and
  // GPU functor), which maps -0.0 to +0.0; the reference's fused spelling
  // `x < 0 ? -x : x` would keep -0.0 and disagree with its own eager path.
  std::string codegen_expr() const override {
    const bool d = is_f64(inputs);
    const auto fn = [&](const char* name) {
      return std::string(name) + (d ? "" : "f") + "({0})";
    };
    switch (op) {
      case LMP_UN_NEG: return "(-{0})";
      case LMP_UN_EXP: return fn("exp");
      case LMP_UN_LOG: return fn("log");
      case LMP_UN_SQRT: return fn("sqrt");
      case LMP_UN_ABS: return fn("fabs");
      case LMP_UN_SIN: return fn("sin");
      case LMP_UN_COS: return fn("cos");
      case LMP_UN_TAN: return fn("tan");
      default:
        return "lmp_clamp({0}, " + float_literal(lo, d) + ", " + float_literal(hi, d) + ")";
    }
  }
};

// Keep-dims reduction over the last axis (see OpKind::Reduce).  The fusion
// backend emits its code itself, replaying the eager row kernel's order.
struct ReduceFn : LazyFunction {
  int op;
  size_t axis;
  ReduceFn(int code, std::vector<std::shared_ptr<TensorImpl>> ins, size_t ax)
      : LazyFunction(std::move(ins)), op(code), axis(ax) {}
  std::shared_ptr<TensorImpl> infer_output() const override {
    OpMeta m = infer_reduct(*inputs[0], axis);
    return std::make_shared<TensorImpl>(Storage(0, inputs[0]->device()), m.shape,
                                        m.dtype);
  }
  bool is_fusible() const override { return true; }
  OpKind kind() const override { return OpKind::Reduce; }
  int code() const override { return op; }
  Scalar param0() const override { return static_cast<Scalar>(axis); }
  void run_eager(TensorImpl& out) override {
    using namespace ops;
    const DeviceType d = inputs[0]->device();
    TensorImpl r = [&]() -> TensorImpl {
      switch (op) {
        case LMP_RED_SUM: return sum_stub()(d, *inputs[0], axis);
        case LMP_RED_MAX: return max_stub()(d, *inputs[0], axis);
        case LMP_RED_MIN: return min_stub()(d, *inputs[0], axis);
        default: return prod_stub()(d, *inputs[0], axis);
      }
    }();
    out.set_realized(r.storage());
  }
  std::string codegen_expr() const override { return ""; }
};

// A constant (full_like under capture).  Fused, it is a literal in the
// generated kernel, so `ones_like(x) * g` costs neither a fill nor its read.
struct FillFn : LazyFunction {
  std::vector<size_t> shape;
  DeviceType dev;
  DataType dt;
  Scalar value;
  FillFn(std::vector<size_t> s, DeviceType d, DataType t, Scalar v)
      : LazyFunction({}), shape(std::move(s)), dev(d), dt(t), value(v) {}
  std::shared_ptr<TensorImpl> infer_output() const override {
    return std::make_shared<TensorImpl>(Storage(0, dev), shape, dt);
  }
  bool is_fusible() const override { return true; }
  OpKind kind() const override { return OpKind::Fill; }
  int code() const override { return 0; }
  Scalar param0() const override { return value; }
  void run_eager(TensorImpl& out) override {
    Storage st(shape_numel(shape) * dtype_size(dt), dev);
    if (st.byte_size()) ops::fill_stub()(dev, st.data(), shape_numel(shape), value, dt);
    out.set_realized(st);
  }
  // The value converted to the tensor's type on the host, as the fill does.
  std::string codegen_expr() const override {
    return float_literal(value, dt == DataType::Float64);
  }
};

}  // namespace

bool is_capture_enabled() { return t_capture; }
void set_capture_enabled(bool enable) { t_capture = enable; }
bool should_capture(DeviceType device) {
  return t_capture && backend(device) != nullptr;
}
CaptureGuard::CaptureGuard(bool enable) : prev_(t_capture) { t_capture = enable; }
CaptureGuard::~CaptureGuard() { t_capture = prev_; }

LazyBackend* backend(DeviceType dev) { return registry()[static_cast<size_t>(dev)]; }
void register_backend(DeviceType dev, LazyBackend* b) {
  registry()[static_cast<size_t>(dev)] = b;
}

std::shared_ptr<TensorImpl> record(std::shared_ptr<LazyFunction> fn) {
  std::shared_ptr<TensorImpl> out = fn->infer_output();
  out->set_deferred(std::move(fn));
  return out;
}

void realize(TensorImpl* t) {
  if (!t->is_deferred()) return;
  LazyBackend* b = backend(t->device());
  LMP_CHECK(b != nullptr) << "no lazy backend registered for device";
  b->realize(t);
}

bool realize_into(TensorImpl* root, const Storage& target) {
  if (!root->is_deferred()) return false;
  LazyBackend* b = backend(root->device());
  LMP_CHECK(b != nullptr) << "no lazy backend registered for device";
  return b->realize_into(root, target);
}

void realize_many(const std::vector<TensorImpl*>& roots,
                  const std::vector<const Storage*>& targets) {
  LMP_CHECK(targets.empty() || targets.size() == roots.size())
      << "realize_many: one target per root";
  std::vector<TensorImpl*> pending;
  std::vector<const Storage*> tg;
  for (size_t i = 0; i < roots.size(); ++i) {
    if (!roots[i]->is_deferred()) continue;
    LMP_CHECK(roots[i]->device() == roots.front()->device())
        << "realize_many: tensors on different devices";
    pending.push_back(roots[i]);
    tg.push_back(targets.empty() ? nullptr : targets[i]);
  }
  if (pending.empty()) return;
  LazyBackend* b = backend(pending.front()->device());
  LMP_CHECK(b != nullptr) << "no lazy backend registered for device";
  b->realize_many(pending, tg);
}

std::shared_ptr<LazyFunction> make_binary(int code, std::shared_ptr<TensorImpl> a,
                                          std::shared_ptr<TensorImpl> b, Scalar p0,
                                          Scalar p1) {
  LMP_CHECK(a->device() == b->device()) << "Tensors are on different devices";
  return std::make_shared<BinaryFn>(
      code, std::vector<std::shared_ptr<TensorImpl>>{std::move(a), std::move(b)}, p0, p1);
}

std::shared_ptr<LazyFunction> make_unary(int code, std::shared_ptr<TensorImpl> a,
                                         Scalar p0, Scalar p1) {
  return std::make_shared<UnaryFn>(code, std::vector<std::shared_ptr<TensorImpl>>{std::move(a)},
                                   p0, p1);
}

std::shared_ptr<LazyFunction> make_fill(const std::vector<size_t>& shape, DeviceType device,
                                        DataType dtype, Scalar value) {
  return std::make_shared<FillFn>(shape, device, dtype, value);
}

std::shared_ptr<LazyFunction> make_reduce(int code, std::shared_ptr<TensorImpl> a,
                                          size_t axis) {
  infer_reduct(*a, axis);  // shape and axis checks, as the eager path does
  return std::make_shared<ReduceFn>(code, std::vector<std::shared_ptr<TensorImpl>>{std::move(a)},
                                    axis);
}

}  // namespace lazy
}  // namespace lmp::tensor
