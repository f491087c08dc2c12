// Registration of the HIP device: `*_hip` adapters for every dispatch-table
// entry the CUDA backend fills (kernels.cu:124-156, memory.cu:97-101,218),
// each a thin shim over the C ABI of liblmp_hip (include/lmp_hip.h).  The CPU
// slot gets storage plumbing only (allocation, fill, copies): arithmetic on
// host tensors is not part of this backend.
#include <cstring>
#include <memory>

#include "ops.hpp"

namespace lmp::tensor::hip {

namespace {

using ops::copy_stub;

int code(DataType t) { return static_cast<int>(t); }

void* mut(const TensorImpl& t) { return const_cast<TensorImpl&>(t).data(); }

void count_launch() { ++backend_stats().eager_launches; }

// ------------------------------------------------------------------ memory

detail::DataPtr empty_hip(size_t bytes) {
  void* p = nullptr;
  hip_ok(lmp_rt_malloc(&p, bytes), "lmp_rt_malloc");
  return detail::DataPtr(p, [](void* q) {
    const int s = lmp_rt_free(q);
    if (s != LMP_OK) throw std::runtime_error(lmp_rt_last_error());
  });
}

void fill_hip(void* ptr, size_t n, Scalar value, DataType t) {
  if (!n) return;
  count_launch();
  hip_ok(lmp_k_fill(code(t), ptr, n, value), "lmp_k_fill");
}

void add_inplace_hip(void* dst, const void* src, size_t n, DataType t) {
  if (!n) return;
  count_launch();
  hip_ok(lmp_k_add_inplace(code(t), dst, src, n), "lmp_k_add_inplace");
}

// Dispatched on the source device (memory.cu:103-174).
void copy_hip(DeviceType to, const void* src, void* dst, size_t n, DataType st,
              DataType dt) {
  if (!n) return;
  if (to == DeviceType::HIP) {
    if (st == dt) hip_ok(lmp_rt_memcpy_d2d(dst, src, n * dtype_size(st)), "memcpy d2d");
    else hip_ok(lmp_k_cast(code(st), code(dt), dst, src, n), "lmp_k_cast");
    return;
  }
  if (st == dt) {
    hip_ok(lmp_rt_memcpy_d2h(dst, src, n * dtype_size(st)), "memcpy d2h");
    return;
  }
  // Convert on the device, then copy the converted buffer down.
  detail::DataPtr tmp = empty_hip(n * dtype_size(dt));
  hip_ok(lmp_k_cast(code(st), code(dt), tmp.data(), src, n), "lmp_k_cast");
  hip_ok(lmp_rt_memcpy_d2h(dst, tmp.data(), n * dtype_size(dt)), "memcpy d2h");
}

detail::DataPtr resize_hip(const detail::DataPtr& old, size_t old_bytes,
                           size_t new_bytes) {
  detail::DataPtr fresh = empty_hip(new_bytes);
  const size_t keep = std::min(old_bytes, new_bytes);
  if (keep) hip_ok(lmp_rt_memcpy_d2d(fresh.data(), old.data(), keep), "memcpy d2d");
  return fresh;
}

// ------------------------------------------------------ host storage only

detail::DataPtr empty_cpu(size_t bytes) {
  char* p = new char[bytes];
  return detail::DataPtr(p, [](void* q) { delete[] static_cast<char*>(q); });
}

void fill_cpu(void* ptr, size_t n, Scalar value, DataType t) {
  visit_dtype(t, [&](auto tag) {
    using T = decltype(tag);
    T* p = static_cast<T*>(ptr);
    const T v = static_cast<T>(value);
    for (size_t i = 0; i < n; ++i) p[i] = v;
  });
}

void convert_host(const void* src, void* dst, size_t n, DataType st, DataType dt) {
  if (st == dt) {
    std::memcpy(dst, src, n * dtype_size(st));
    return;
  }
  visit_dtype(st, [&](auto stag) {
    using S = decltype(stag);
    visit_dtype(dt, [&](auto dtag) {
      using D = decltype(dtag);
      const S* s = static_cast<const S*>(src);
      D* d = static_cast<D*>(dst);
      for (size_t i = 0; i < n; ++i) d[i] = static_cast<D>(s[i]);
    });
  });
}

void copy_cpu(DeviceType to, const void* src, void* dst, size_t n, DataType st,
              DataType dt) {
  if (!n) return;
  if (to == DeviceType::CPU) {
    convert_host(src, dst, n, st, dt);
    return;
  }
  // A single value (Python scalars become [1] tensors) goes down as a kernel
  // argument of a fill launch: stream-ordered, no host synchronisation.  The
  // host-side conversion to the destination dtype equals the device cast.
  if (n == 1 && st != DataType::Int64) {
    double v = 0;
    convert_host(src, &v, 1, st, DataType::Float64);
    count_launch();
    hip_ok(lmp_k_fill(code(dt), dst, 1, v), "lmp_k_fill");
    return;
  }
  if (st == dt) {
    hip_ok(lmp_rt_memcpy_h2d(dst, src, n * dtype_size(st)), "memcpy h2d");
    return;
  }
  // Upload in the source dtype, convert on the device (memory.cu:103-127).
  detail::DataPtr tmp = empty_hip(n * dtype_size(st));
  hip_ok(lmp_rt_memcpy_h2d(tmp.data(), src, n * dtype_size(st)), "memcpy h2d");
  hip_ok(lmp_k_cast(code(st), code(dt), dst, tmp.data(), n), "lmp_k_cast");
}

detail::DataPtr resize_cpu(const detail::DataPtr& old, size_t old_bytes,
                           size_t new_bytes) {
  detail::DataPtr fresh = empty_cpu(new_bytes);
  const size_t keep = std::min(old_bytes, new_bytes);
  if (keep) std::memcpy(fresh.data(), old.data(), keep);
  return fresh;
}

void add_inplace_cpu(void*, const void*, size_t, DataType) {
  throw std::runtime_error(
      "add_inplace on CPU tensors: this build provides the HIP device backend "
      "only; move the tensors to device.hip");
}

// -------------------------------------------------------------- elementwise

// Bring an input to the op's output dtype (cast-then-operate order of
// cpu/ptr_pack.hpp:9-35); returns the same storage when no cast is needed.
Storage as_dtype(const TensorImpl& t, DataType dt, void** ptr) {
  void* p = mut(t);
  if (t.type() == dt) {
    *ptr = p;
    return t.storage();
  }
  Storage s(t.numel() * dtype_size(dt), DeviceType::HIP);
  if (t.numel()) {
    count_launch();
    hip_ok(lmp_k_cast(code(t.type()), code(dt), s.data(), p, t.numel()), "lmp_k_cast");
  }
  *ptr = s.data();
  return s;
}

TensorImpl run_binary(int op, const TensorImpl& a, const TensorImpl& b, Scalar p0 = 0,
                      Scalar p1 = 0) {
  OpMeta m = infer_binary(a, b);
  void *pa = nullptr, *pb = nullptr;
  Storage ka = as_dtype(a, m.dtype, &pa);
  Storage kb = as_dtype(b, m.dtype, &pb);
  Storage out(m.size * dtype_size(m.dtype), DeviceType::HIP);
  if (m.size) {
    lmp_bcast d{};
    d.ndim = static_cast<int32_t>(m.shape.size());
    const std::vector<stride_t> sa = padded_strides(a.shape(), m.shape.size());
    const std::vector<stride_t> sb = padded_strides(b.shape(), m.shape.size());
    for (size_t i = 0; i < m.shape.size(); ++i) {
      d.shape[i] = static_cast<int64_t>(m.shape[i]);
      d.stride_a[i] = sa[i];
      d.stride_b[i] = sb[i];
    }
    count_launch();
    hip_ok(lmp_k_binary(op, code(m.dtype), out.data(), pa, pb, &d, p0, p1),
           "lmp_k_binary");
  }
  return TensorImpl(out, m.shape, m.dtype);
}

template <int OP>
TensorImpl binary_hip(const TensorImpl& a, const TensorImpl& b) {
  return run_binary(OP, a, b);
}

TensorImpl run_unary(int op, const TensorImpl& a, Scalar p0 = 0, Scalar p1 = 0) {
  Storage out(a.nbytes(), DeviceType::HIP);
  if (a.numel()) {
    void* in = mut(a);
    count_launch();
    hip_ok(lmp_k_unary(op, code(a.type()), out.data(), in, a.numel(), p0, p1),
           "lmp_k_unary");
  }
  return TensorImpl(out, a.shape(), a.type());
}

template <int OP>
TensorImpl unary_hip(const TensorImpl& a) {
  return run_unary(OP, a);
}

TensorImpl clamp_hip(const TensorImpl& a, Scalar lo, Scalar hi) {
  return run_unary(LMP_UN_CLAMP, a, lo, hi);
}

TensorImpl abs_backward_hip(const TensorImpl& x, const TensorImpl& g) {
  return run_binary(LMP_BIN_ABS_BACKWARD, x, g);
}

TensorImpl clamp_backward_hip(const TensorImpl& x, const TensorImpl& g, Scalar lo,
                              Scalar hi) {
  return run_binary(LMP_BIN_CLAMP_BACKWARD, x, g, lo, hi);
}

// --------------------------------------------------------------- reductions

template <int OP>
TensorImpl reduce_hip(const TensorImpl& a, size_t axis) {
  OpMeta m = infer_reduct(a, axis);
  Storage out(m.size * dtype_size(m.dtype), DeviceType::HIP);
  if (m.size) {
    size_t outer = 1, inner = 1;
    for (size_t i = 0; i < axis; ++i) outer *= a.shape()[i];
    for (size_t i = axis + 1; i < a.shape().size(); ++i) inner *= a.shape()[i];
    void* in = mut(a);
    count_launch();
    hip_ok(lmp_k_reduce(OP, code(a.type()), out.data(), in, outer, a.shape()[axis],
                        inner),
           "lmp_k_reduce");
  }
  return TensorImpl(out, m.shape, m.dtype);
}

// ------------------------------------------------------------------- matrix

struct GemmShape {
  size_t m, n, k;
};

GemmShape gemm_shape(const TensorImpl& a, const TensorImpl& b, bool ta, bool tb) {
  LMP_CHECK(a.shape().size() == 2 && b.shape().size() == 2)
      << "Both matrices must be 2D.";
  const size_t m = ta ? a.shape()[1] : a.shape()[0];
  const size_t k = ta ? a.shape()[0] : a.shape()[1];
  const size_t kb = tb ? b.shape()[1] : b.shape()[0];
  const size_t n = tb ? b.shape()[0] : b.shape()[1];
  LMP_CHECK(k == kb) << "Incompatible matrix dimensions for multiplication.";
  return {m, n, k};
}

// C (+)= op(A) op(B) in dtype `dt`; A and B are cast to `dt` first, as the
// reference's matmul casts each operand to the output type
// (cpu/matrix.cpp:14-15).
void gemm_into(void* c, DataType dt, const TensorImpl& a, const TensorImpl& b, bool ta,
               bool tb, const GemmShape& s, bool accumulate) {
  if (!s.m || !s.n) return;
  HostTimer timer(&backend_stats().gemm_host_ns);
  void *pa = nullptr, *pb = nullptr;
  Storage ka = as_dtype(a, dt, &pa);
  Storage kb = as_dtype(b, dt, &pb);
  count_launch();
  hip_ok(lmp_k_gemm(code(dt), ta, tb, s.m, s.n, s.k, pa, a.shape()[1], pb, b.shape()[1], c,
                    s.n, accumulate ? 1 : 0),
         "lmp_k_gemm");
}

TensorImpl gemm_hip(const TensorImpl& a, const TensorImpl& b, bool ta, bool tb) {
  const GemmShape s = gemm_shape(a, b, ta, tb);
  const DataType dt = type_upcast(a.type(), b.type());
  Storage out(s.m * s.n * dtype_size(dt), DeviceType::HIP);
  gemm_into(out.data(), dt, a, b, ta, tb, s, false);
  return TensorImpl(out, {s.m, s.n}, dt);
}

TensorImpl matmul_hip(const TensorImpl& a, const TensorImpl& b) {
  return gemm_hip(a, b, false, false);
}

TensorImpl matmul_t_hip(const TensorImpl& a, const TensorImpl& b, bool ta, bool tb) {
  return gemm_hip(a, b, ta, tb);
}

// c += op(a) op(b) for a gradient c, accumulated by the GEMM.  The product's
// promoted dtype must be c's, as add_inplace requires identical dtypes
// (native/memory_ops.cpp:28-35).
void matmul_acc_hip(TensorImpl& c, const TensorImpl& a, const TensorImpl& b, bool ta,
                    bool tb) {
  const GemmShape s = gemm_shape(a, b, ta, tb);
  LMP_CHECK(c.shape().size() == 2 && c.shape()[0] == s.m && c.shape()[1] == s.n)
      << "add_inplace requires tensors with identical shapes";
  const DataType dt = type_upcast(a.type(), b.type());
  LMP_CHECK(dt == c.type()) << "add_inplace requires tensors with identical dtypes";
  gemm_into(c.data(), dt, a, b, ta, tb, s, true);
}

void matmul_colsum_hip(const TensorImpl& a, const TensorImpl& b, bool ta, bool tb,
                       TensorImpl& c, bool acc_c, TensorImpl& s, bool acc_s) {
  const GemmShape sh = gemm_shape(a, b, ta, tb);
  LMP_CHECK(c.shape().size() == 2 && c.shape()[0] == sh.m && c.shape()[1] == sh.n)
      << "add_inplace requires tensors with identical shapes";
  LMP_CHECK(s.numel() == sh.n) << "add_inplace requires tensors with identical shapes";
  if (!sh.m || !sh.n) return;
  HostTimer timer(&backend_stats().gemm_host_ns);
  const void* pa = mut(a);
  const void* pb = mut(b);
  void* pc = c.data();
  void* ps = s.data();
  count_launch();
  hip_ok(lmp_k_gemm_colsum_f32(ta, tb, sh.m, sh.n, sh.k, static_cast<const float*>(pa),
                               a.shape()[1], static_cast<const float*>(pb), b.shape()[1],
                               static_cast<float*>(pc), sh.n, acc_c ? 1 : 0,
                               static_cast<float*>(ps), acc_s ? 1 : 0),
         "lmp_k_gemm_colsum_f32");
}

void matmul_colsum_masked_hip(const TensorImpl& a, const TensorImpl& b, const TensorImpl& mask,
                              bool ta, TensorImpl& c, bool acc_c, TensorImpl& s, bool acc_s) {
  const GemmShape sh = gemm_shape(a, b, ta, false);
  LMP_CHECK(c.shape().size() == 2 && c.shape()[0] == sh.m && c.shape()[1] == sh.n)
      << "add_inplace requires tensors with identical shapes";
  LMP_CHECK(s.numel() == sh.n) << "add_inplace requires tensors with identical shapes";
  if (!sh.m || !sh.n) return;
  HostTimer timer(&backend_stats().gemm_host_ns);
  const void* pa = mut(a);
  const void* pb = mut(b);
  const void* pm = mut(mask);
  void* pc = c.data();
  void* ps = s.data();
  // One launch in the tiny-GEMM range (K <= 512, at most 2^21 multiply-adds),
  // where the mask is applied as B is loaded; otherwise the mask kernel too.
  count_launch();
  if (sh.k > 512 || double(sh.m) * double(sh.n) * double(sh.k) > double(1 << 21)) count_launch();
  hip_ok(lmp_k_gemm_colsum_masked_f32(ta, sh.m, sh.n, sh.k, static_cast<const float*>(pa),
                                      a.shape()[1], static_cast<const float*>(pb),
                                      static_cast<const float*>(pm), b.shape()[1],
                                      static_cast<float*>(pc), sh.n, acc_c ? 1 : 0,
                                      static_cast<float*>(ps), acc_s ? 1 : 0),
         "lmp_k_gemm_colsum_masked_f32");
}

// Whether lmp_k_linear_backward_f32 runs both products on the tiny GEMM's
// 16 x 16 blocks in one launch (K <= 512, at most 2^21 multiply-adds, and
// 32 x 32 blocks short of a quarter of the CUs), for the launch count.
bool linear_backward_one_launch(size_t batch, size_t in, size_t out) {
  static const int cu = [] {
    lmp_rt_info info{};
    return lmp_rt_device_info(&info) == LMP_OK ? int(info.cu_count) : 0;
  }();
  const auto tiny16 = [](size_t m, size_t n, size_t k) {
    return k <= 512 && double(m) * double(n) * double(k) <= double(1 << 21) &&
           double((m + 31) / 32) * double((n + 31) / 32) * 4 < double(cu);
  };
  return tiny16(in, out, batch) && tiny16(batch, in, out);
}

void linear_backward_hip(const TensorImpl& x, const TensorImpl& w, const TensorImpl& g,
                         TensorImpl& dx, bool acc_dx, TensorImpl& dw, bool acc_dw,
                         TensorImpl& db, bool acc_db) {
  const size_t batch = x.shape()[0], in = x.shape()[1], out = w.shape()[1];
  LMP_CHECK(dx.shape().size() == 2 && dx.shape()[0] == batch && dx.shape()[1] == in)
      << "add_inplace requires tensors with identical shapes";
  LMP_CHECK(dw.shape().size() == 2 && dw.shape()[0] == in && dw.shape()[1] == out)
      << "add_inplace requires tensors with identical shapes";
  LMP_CHECK(db.numel() == out) << "add_inplace requires tensors with identical shapes";
  HostTimer timer(&backend_stats().gemm_host_ns);
  const void* px = mut(x);
  const void* pw = mut(w);
  const void* pg = mut(g);
  count_launch();
  if (!linear_backward_one_launch(batch, in, out)) count_launch();
  hip_ok(lmp_k_linear_backward_f32(batch, in, out, static_cast<const float*>(px), in,
                                   static_cast<const float*>(pw), out,
                                   static_cast<const float*>(pg), out,
                                   static_cast<float*>(dx.data()), in, acc_dx ? 1 : 0,
                                   static_cast<float*>(dw.data()), out, acc_dw ? 1 : 0,
                                   static_cast<float*>(db.data()), acc_db ? 1 : 0),
         "lmp_k_linear_backward_f32");
}

TensorImpl linear_hip(const TensorImpl& x, const TensorImpl& w, const TensorImpl& b,
                      bool relu) {
  const GemmShape s = gemm_shape(x, w, false, false);
  Storage out(s.m * s.n * sizeof(float), DeviceType::HIP);
  if (s.m && s.n) {
    HostTimer timer(&backend_stats().gemm_host_ns);
    const void* px = mut(x);
    const void* pw = mut(w);
    const void* pb = mut(b);
    count_launch();
    const auto entry = relu ? lmp_k_linear_relu_f32 : lmp_k_linear_f32;
    hip_ok(entry(0, 0, s.m, s.n, s.k, static_cast<const float*>(px), s.k,
                 static_cast<const float*>(pw), s.n, static_cast<const float*>(pb),
                 static_cast<float*>(out.data()), s.n),
           relu ? "lmp_k_linear_relu_f32" : "lmp_k_linear_f32");
  }
  return TensorImpl(out, {s.m, s.n}, DataType::Float32);
}

TensorImpl transpose_hip(const TensorImpl& a) {
  LMP_CHECK(a.shape().size() == 2)
      << "Invalid argument, transpose can only be performed on matrices of dim 2";
  const size_t m = a.shape()[0], n = a.shape()[1];
  Storage out(a.nbytes(), DeviceType::HIP);
  if (a.numel()) {
    void* in = mut(a);
    count_launch();
    hip_ok(lmp_k_transpose(code(a.type()), out.data(), in, m, n), "lmp_k_transpose");
  }
  return TensorImpl(out, {n, m}, a.type());
}

}  // namespace

using namespace ops;
constexpr DeviceType kHip = DeviceType::HIP;
constexpr DeviceType kCpu = DeviceType::CPU;

LMP_REGISTER_DISPATCH(empty_stub, kHip, empty_hip)
LMP_REGISTER_DISPATCH(fill_stub, kHip, fill_hip)
LMP_REGISTER_DISPATCH(copy_stub, kHip, copy_hip)
LMP_REGISTER_DISPATCH(resize_stub, kHip, resize_hip)
LMP_REGISTER_DISPATCH(add_inplace_stub, kHip, add_inplace_hip)
LMP_REGISTER_DISPATCH(empty_stub, kCpu, empty_cpu)
LMP_REGISTER_DISPATCH(fill_stub, kCpu, fill_cpu)
LMP_REGISTER_DISPATCH(copy_stub, kCpu, copy_cpu)
LMP_REGISTER_DISPATCH(resize_stub, kCpu, resize_cpu)
LMP_REGISTER_DISPATCH(add_inplace_stub, kCpu, add_inplace_cpu)

// Binary, unary, reductions: one instantiation per op code.
#define LMP_REG_BIN(name, CODE)                                   \
  static const binary_fn name##_hip = &binary_hip<CODE>;          \
  LMP_REGISTER_DISPATCH(name##_stub, kHip, name##_hip)
LMP_REG_BIN(add, LMP_BIN_ADD)
LMP_REG_BIN(sub, LMP_BIN_SUB)
LMP_REG_BIN(mul, LMP_BIN_MUL)
LMP_REG_BIN(div, LMP_BIN_DIV)
LMP_REG_BIN(pow, LMP_BIN_POW)
LMP_REG_BIN(eq, LMP_BIN_EQ)
LMP_REG_BIN(ne, LMP_BIN_NE)
LMP_REG_BIN(ge, LMP_BIN_GE)
LMP_REG_BIN(le, LMP_BIN_LE)
LMP_REG_BIN(gt, LMP_BIN_GT)
LMP_REG_BIN(lt, LMP_BIN_LT)
#undef LMP_REG_BIN

#define LMP_REG_UN(name, CODE)                                    \
  static const unary_fn name##_hip = &unary_hip<CODE>;            \
  LMP_REGISTER_DISPATCH(name##_stub, kHip, name##_hip)
LMP_REG_UN(neg, LMP_UN_NEG)
LMP_REG_UN(exp, LMP_UN_EXP)
LMP_REG_UN(log, LMP_UN_LOG)
LMP_REG_UN(sqrt, LMP_UN_SQRT)
LMP_REG_UN(abs, LMP_UN_ABS)
LMP_REG_UN(sin, LMP_UN_SIN)
LMP_REG_UN(cos, LMP_UN_COS)
LMP_REG_UN(tan, LMP_UN_TAN)
#undef LMP_REG_UN

#define LMP_REG_RED(name, CODE)                                   \
  static const reduct_fn name##_hip = &reduce_hip<CODE>;          \
  LMP_REGISTER_DISPATCH(name##_stub, kHip, name##_hip)
LMP_REG_RED(sum, LMP_RED_SUM)
LMP_REG_RED(max, LMP_RED_MAX)
LMP_REG_RED(min, LMP_RED_MIN)
LMP_REG_RED(prod, LMP_RED_PROD)
#undef LMP_REG_RED

LMP_REGISTER_DISPATCH(clamp_stub, kHip, clamp_hip)
LMP_REGISTER_DISPATCH(abs_backward_stub, kHip, abs_backward_hip)
LMP_REGISTER_DISPATCH(clamp_backward_stub, kHip, clamp_backward_hip)
LMP_REGISTER_DISPATCH(matmul_stub, kHip, matmul_hip)
LMP_REGISTER_DISPATCH(matmul_t_stub, kHip, matmul_t_hip)
LMP_REGISTER_DISPATCH(matmul_acc_stub, kHip, matmul_acc_hip)
LMP_REGISTER_DISPATCH(linear_stub, kHip, linear_hip)
LMP_REGISTER_DISPATCH(matmul_colsum_stub, kHip, matmul_colsum_hip)
LMP_REGISTER_DISPATCH(matmul_colsum_masked_stub, kHip, matmul_colsum_masked_hip)
LMP_REGISTER_DISPATCH(linear_backward_stub, kHip, linear_backward_hip)
LMP_REGISTER_DISPATCH(transpose_stub, kHip, transpose_hip)

}  // namespace lmp::tensor::hip
