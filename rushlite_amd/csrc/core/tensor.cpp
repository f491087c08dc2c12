// Storage, TensorImpl and Tensor (Lamp3: storage.cpp, tensor_impl.cpp,
// tensor.cpp, utils/fill_like.cpp, infer_meta.cpp, utils/align_utils.cpp).
#include "tensor.hpp"

#include <algorithm>
#include <cstring>
#include <iostream>
#include <map>
#include <mutex>
#include <tuple>

#include "ops.hpp"

namespace lmp {

void hip_throw(int status, const char* what) {
  std::string msg = std::string(what) + " failed (status " +
                    std::to_string(status) + "): " + lmp_rt_last_error();
  throw std::runtime_error(msg);
}

namespace tensor {

const char* dtype_name(DataType t) {
  switch (t) {
    case DataType::Bool: return "Bool";
    case DataType::Int16: return "Int16";
    case DataType::Int32: return "Int32";
    case DataType::Int64: return "Int64";
    case DataType::Float32: return "Float32";
    case DataType::Float64: return "Float64";
  }
  return "Unknown";
}

const char* device_name(DeviceType d) {
  switch (d) {
    case DeviceType::CPU: return "CPU";
    case DeviceType::HIP: return "HIP";
    default: return "Unknown";
  }
}

std::ostream& operator<<(std::ostream& os, DataType t) { return os << dtype_name(t); }
std::ostream& operator<<(std::ostream& os, DeviceType d) { return os << device_name(d); }

std::ostream& operator<<(std::ostream& os, const std::vector<size_t>& v) {
  os << "[";
  for (size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << v[i];
  return os << "]";
}

size_t shape_numel(const std::vector<size_t>& shape) {
  if (shape.empty()) return 0;  // tensor_impl.cpp:20-22: empty shape, no data
  size_t n = 1;
  for (size_t s : shape) n *= s;
  return n;
}

namespace ops {
LMP_DEFINE_DISPATCH(copy_fn, copy_stub)
LMP_DEFINE_DISPATCH(empty_fn, empty_stub)
LMP_DEFINE_DISPATCH(fill_fn, fill_stub)
LMP_DEFINE_DISPATCH(resize_fn, resize_stub)
LMP_DEFINE_DISPATCH(add_inplace_fn, add_inplace_stub)
}  // namespace ops

// ------------------------------------------------------------------ DataPtr

detail::DataPtr::DataPtr(void* p, std::function<void(void*)> deleter)
    : ptr(p, [d = std::move(deleter)](void* q) {
        try {
          d(q);
        } catch (const std::exception& e) {
          std::cerr << "DataPtr deleter error: " << e.what() << "\n";
        } catch (...) {
          std::cerr << "DataPtr deleter threw a non-std exception\n";
        }
      }) {}

// ------------------------------------------------------------------ Storage

struct Storage::Impl {
  detail::DataPtr ptr;
  size_t bytes;
  DeviceType device;
};

Storage::Storage(size_t byte_size, DeviceType device)
    : impl_(std::make_shared<Impl>(
          Impl{byte_size ? ops::empty_stub()(device, byte_size) : detail::DataPtr(),
               byte_size, device})) {}

void* Storage::data() const noexcept { return impl_->ptr.data(); }
size_t Storage::byte_size() const noexcept { return impl_->bytes; }
DeviceType Storage::device() const noexcept { return impl_->device; }

void Storage::resize(size_t new_bytes) {
  impl_->ptr = ops::resize_stub()(impl_->device, impl_->ptr, impl_->bytes, new_bytes);
  impl_->bytes = new_bytes;
}

// --------------------------------------------------------------- TensorImpl

TensorImpl::TensorImpl(const void* host, size_t count, DataType host_type,
                       const std::vector<size_t>& shape, DeviceType device,
                       DataType dtype)
    : storage_(shape_numel(shape) * dtype_size(dtype), device),
      shape_(shape),
      type_(dtype),
      numel_(shape_numel(shape)) {
  LMP_CHECK(count == numel_)
      << "Size mismatch, product of shape must equal num elements";
  if (numel_)
    ops::copy_stub()(DeviceType::CPU, device, host, storage_.data(), numel_,
                     host_type, type_);
  compute_strides();
}

TensorImpl::TensorImpl(Storage storage, const std::vector<size_t>& shape,
                       DataType dtype)
    : storage_(std::move(storage)), shape_(shape), type_(dtype),
      numel_(shape_numel(shape)) {
  LMP_CHECK(storage_.byte_size() == 0 ||
            storage_.byte_size() / dtype_size(dtype) == numel_)
      << "Storage size mismatch: expected " << numel_ << " elements of "
      << dtype << ", storage has " << storage_.byte_size() << " bytes";
  compute_strides();
}

void TensorImpl::compute_strides() {
  strides_.assign(shape_.size(), 0);
  stride_t s = 1;
  for (size_t i = shape_.size(); i-- > 0;) {
    strides_[i] = s;
    s *= static_cast<stride_t>(shape_[i]);
  }
}

void* TensorImpl::data() {
  if (is_deferred()) lazy::realize(this);
  return storage_.data();
}

void TensorImpl::set_realized(Storage storage) {
  LMP_CHECK(storage.byte_size() == nbytes())
      << "set_realized: storage size mismatch: expected " << nbytes()
      << " bytes, got " << storage.byte_size();
  LMP_CHECK(storage.device() == storage_.device()) << "set_realized: device mismatch";
  storage_ = std::move(storage);
  lazy_.reset();
}

void TensorImpl::set_deferred(std::shared_ptr<lazy::LazyFunction> op) {
  LMP_CHECK(!is_deferred()) << "tensor already has a pending op";
  lazy_ = std::move(op);
}

void TensorImpl::replace_pending_constant(std::shared_ptr<lazy::LazyFunction> op) {
  LMP_CHECK(is_deferred() && lazy_->inputs.empty())
      << "replace_pending_constant: tensor is not a pending constant";
  lazy_ = std::move(op);
}

// Views share storage.  A pending graph is realised first so that the view
// and its base read the same buffer instead of each re-running the graph.
TensorImpl TensorImpl::reshape(std::vector<size_t> new_shape) {
  LMP_CHECK(shape_numel(new_shape) == numel_)
      << "Cannot reshape tensor: total number of elements must remain the same.";
  data();
  TensorImpl v(*this);
  v.shape_ = std::move(new_shape);
  v.compute_strides();
  return v;
}

TensorImpl TensorImpl::squeeze(size_t dim) {
  LMP_CHECK(dim < shape_.size()) << "Dimension out of range for squeeze";
  LMP_CHECK(shape_[dim] == 1) << "Cannot squeeze dimension that is not size 1";
  data();
  TensorImpl v(*this);
  v.shape_.erase(v.shape_.begin() + static_cast<long>(dim));
  v.compute_strides();
  return v;
}

TensorImpl TensorImpl::expand_dims(size_t dim) {
  LMP_CHECK(dim <= shape_.size()) << "Dimension out of range for expand_dims";
  data();
  TensorImpl v(*this);
  v.shape_.insert(v.shape_.begin() + static_cast<long>(dim), 1);
  v.compute_strides();
  return v;
}

Scalar TensorImpl::index(const std::vector<size_t>& idx) {
  LMP_CHECK(idx.size() == shape_.size()) << "Indexing does not match shape";
  size_t at = 0;
  for (size_t i = 0; i < idx.size(); ++i) {
    LMP_CHECK(idx[i] < shape_[i]) << "Index out of range";
    at += static_cast<size_t>(strides_[i]) * idx[i];
  }
  char* base = static_cast<char*>(data()) + at * dtype_size(type_);
  double out = 0;
  ops::copy_stub()(device(), DeviceType::CPU, base, &out, 1, type_, DataType::Float64);
  return out;
}

void TensorImpl::copy(TensorImpl& other) {
  LMP_CHECK(other.numel() == numel_) << "copy: element counts differ";
  void* src = other.data();
  data();
  ops::copy_stub()(other.device(), device(), src, storage_.data(), numel_,
                   other.type(), type_);
}

void TensorImpl::fill(Scalar value) {
  data();
  if (numel_) ops::fill_stub()(device(), storage_.data(), numel_, value, type_);
}

void TensorImpl::print(std::ostream& os) {
  constexpr size_t kMaxPrint = 20;  // tensor_impl.cpp:138-165
  const size_t n = std::min(kMaxPrint, numel_);
  std::vector<double> vals(n);
  if (n) {
    void* src = data();
    ops::copy_stub()(device(), DeviceType::CPU, src, vals.data(), n, type_,
                     DataType::Float64);
  }
  os << "Tensor(data=[";
  for (size_t i = 0; i < n; ++i) {
    os << vals[i];
    if (i + 1 < n) os << ", ";
    else if (n < numel_) os << ",...";
  }
  os << "], shape=[";
  for (size_t i = 0; i < shape_.size(); ++i) os << (i ? ", " : "") << shape_[i];
  os << "], dtype=" << type_ << ", device=" << device() << ")";
}

// ------------------------------------------------------------------- Tensor

void* Tensor::data() { return impl_->data(); }

void Tensor::copy_to_host(void* dst, DataType dst_type) const {
  if (!impl_->numel()) return;
  void* src = impl_->data();
  ops::copy_stub()(device(), DeviceType::CPU, src, dst, numel(), type(), dst_type);
}

Tensor Tensor::reshape(std::vector<size_t> s) const { return ops::reshape(*this, std::move(s)); }
Tensor Tensor::squeeze(size_t d) const { return ops::squeeze(*this, d); }
Tensor Tensor::expand_dims(size_t d) const { return ops::expand_dims(*this, d); }
Tensor Tensor::to(DeviceType d) const { return ops::to(*this, d); }
void Tensor::copy(const Tensor& other) { impl_->copy(*other.impl_); }
void Tensor::fill(Scalar v) { impl_->fill(v); }
void Tensor::realize() { impl_->data(); }

std::ostream& operator<<(std::ostream& os, const Tensor& t) {
  t.impl_->print(os);
  return os;
}

Tensor empty(const std::vector<size_t>& shape, DeviceType device, DataType dtype) {
  Storage st(shape_numel(shape) * dtype_size(dtype), device);
  return detail::UnsafeTensorAccessor::fromImpl(
      std::make_shared<TensorImpl>(st, shape, dtype));
}

Tensor full_like(const Tensor& t, Scalar value) {
  // Under capture a float constant stays pending, so a consumer region can
  // take it as a literal (fill_like.cpp:8-20 fills eagerly).
  if (lazy::should_capture(t.device()) &&
      (t.type() == DataType::Float32 || t.type() == DataType::Float64) && t.numel() > 0)
    return detail::UnsafeTensorAccessor::fromImpl(
        lazy::record(lazy::make_fill(t.shape(), t.device(), t.type(), value)));
  Tensor out = empty(t.shape(), t.device(), t.type());
  out.fill(value);
  return out;
}
Tensor ones_like(const Tensor& t) { return full_like(t, 1); }
Tensor zeros_like(const Tensor& t) { return full_like(t, 0); }

// Scalars in expressions (`x + 1e-3`) are [1] tensors of the operand's dtype
// and device (native/overloads.hpp:16-28).  They are internal, never handed
// to the user and never written in place, so each distinct (device, dtype,
// value) is built once and shared; a training loop then issues no upload per
// scalar per step.
//
// While a device graph is captured the value upload is only recorded, so a
// scalar first made then stays out of the cache; every scalar the capture uses
// is also kept in the graph's keep-alive list, since its buffer is read by
// each replay.
namespace {
std::mutex g_scalar_mu;
std::vector<Tensor>* g_graph_keep = nullptr;
}  // namespace

void set_graph_keep_alive(std::vector<Tensor>* keep) {
  std::lock_guard<std::mutex> lock(g_scalar_mu);
  g_graph_keep = keep;
}

Tensor scalar_like(const Tensor& t, Scalar s) {
  using Key = std::tuple<uint64_t, size_t, int>;
  static auto* cache = new std::map<Key, Tensor>();  // outlives static teardown
  uint64_t bits;
  std::memcpy(&bits, &s, sizeof bits);
  const Key key{bits, static_cast<size_t>(t.device()), static_cast<int>(t.type())};
  std::lock_guard<std::mutex> lock(g_scalar_mu);
  auto it = cache->find(key);
  if (it != cache->end()) {
    if (g_graph_keep) g_graph_keep->push_back(it->second);
    return it->second;
  }
  Tensor fresh(std::vector<Scalar>{s}, {1}, t.device(), t.type());
  if (g_graph_keep) {
    g_graph_keep->push_back(fresh);
    return fresh;
  }
  if (cache->size() >= 4096) cache->clear();
  cache->emplace(key, fresh);
  return fresh;
}

// ----------------------------------------------------------------- metadata

std::vector<size_t> broadcast_shapes(const std::vector<size_t>& a,
                                     const std::vector<size_t>& b) {
  const size_t nd = std::max(a.size(), b.size());
  LMP_CHECK(nd <= kMaxDims) << "Too many dims";
  std::vector<size_t> out(nd);
  for (size_t i = 0; i < nd; ++i) {
    const size_t off = nd - 1 - i;
    const size_t av = off < a.size() ? a[a.size() - 1 - off] : 1;
    const size_t bv = off < b.size() ? b[b.size() - 1 - off] : 1;
    LMP_CHECK(av == 1 || bv == 1 || av == bv)
        << "calc_aligned_shape: Broadcast rule violation.";
    out[i] = av != 1 ? av : bv;
  }
  return out;
}

std::vector<stride_t> padded_strides(const std::vector<size_t>& in, size_t nd) {
  std::vector<stride_t> out(nd, 0);
  stride_t s = 1;
  for (size_t k = 0; k < in.size(); ++k) {
    const size_t src = in.size() - 1 - k;
    if (in[src] != 1) out[nd - 1 - k] = s;
    s *= static_cast<stride_t>(in[src]);
  }
  return out;
}

OpMeta infer_unary(const TensorImpl& a) {
  return {a.type(), a.shape(), a.numel(), false};
}

OpMeta infer_binary(const TensorImpl& a, const TensorImpl& b) {
  LMP_CHECK(a.device() == b.device()) << "Tensors are on different devices";
  OpMeta m{type_upcast(a.type(), b.type()), a.shape(), a.numel(), false};
  if (a.shape() != b.shape()) {
    m.expand = true;
    m.shape = broadcast_shapes(a.shape(), b.shape());
    m.size = shape_numel(m.shape);
  }
  return m;
}

OpMeta infer_reduct(const TensorImpl& a, size_t axis) {
  LMP_CHECK(axis < a.shape().size()) << "Axis out of range for reduction";
  OpMeta m{a.type(), a.shape(), a.numel(), false};
  m.size = a.shape()[axis] ? m.size / a.shape()[axis] : 0;
  m.shape[axis] = 1;
  if (a.shape()[axis] == 0) m.size = shape_numel(m.shape);
  return m;
}

}  // namespace tensor
}  // namespace lmp
