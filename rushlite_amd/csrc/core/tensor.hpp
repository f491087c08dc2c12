// Tensor core of the host framework: DataPtr, Storage, TensorImpl, Tensor and
// the per-device dispatch tables the device backends register into.
//
// Interface follows Lamp3 (tensor/tensor.hpp:29-102, tensor_impl.hpp:32-115,
// storage.hpp:34-69, data_ptr.hpp:22-38, dispatch_stub.hpp:21-64) so a
// backend written against those tables plugs in unchanged.
#pragma once

#include <array>
#include <functional>
#include <memory>
#include <numeric>
#include <ostream>
#include <string>
#include <utility>
#include <vector>

#include "common.hpp"

namespace lmp::tensor {

class TensorImpl;
namespace lazy {
struct LazyFunction;
}

namespace detail {

// Per-device function-pointer table (dispatch_stub.hpp:21-64).
template <typename Fn>
class DispatchStub {
 public:
  using fn_type = Fn;
  void register_kernel(DeviceType dev, Fn f) { table_[index(dev)] = f; }
  bool has(DeviceType dev) const { return table_[index(dev)] != nullptr; }
  template <typename... Args>
  decltype(auto) operator()(DeviceType dev, Args&&... args) const {
    Fn f = table_[index(dev)];
    LMP_CHECK(f != nullptr) << "Kernel for this backend not registered (device "
                            << device_name(dev) << ")";
    return f(std::forward<Args>(args)...);
  }

 private:
  static size_t index(DeviceType dev) { return static_cast<size_t>(dev); }
  std::array<Fn, static_cast<size_t>(DeviceType::Count)> table_{};
};

// Owning pointer with a type-erased deleter; deleter failures are reported,
// never thrown from a destructor (data_ptr.hpp:26-35).
struct DataPtr {
  std::shared_ptr<void> ptr;
  DataPtr() = default;
  DataPtr(void* p, std::function<void(void*)> deleter);
  void* data() const { return ptr.get(); }
};

}  // namespace detail

#define LMP_DECLARE_DISPATCH(fn_type, stub_name) \
  ::lmp::tensor::detail::DispatchStub<fn_type>& stub_name();

#define LMP_DEFINE_DISPATCH(fn_type, stub_name)               \
  ::lmp::tensor::detail::DispatchStub<fn_type>& stub_name() { \
    static ::lmp::tensor::detail::DispatchStub<fn_type> s;    \
    return s;                                                 \
  }

#define LMP_REGISTER_DISPATCH(stub_name, dev, kernel_fn)                \
  namespace {                                                           \
  const bool _lmp_reg_##kernel_fn = [] {                                \
    stub_name().register_kernel(dev, kernel_fn);                        \
    return true;                                                        \
  }();                                                                  \
  }

namespace ops {
// Memory entry points (native/memory_ops.hpp:14-25).  copy is dispatched on
// the SOURCE device and told the destination device.
using copy_fn = void (*)(DeviceType to, const void* src, void* dst, size_t n,
                         DataType src_t, DataType dst_t);
using empty_fn = detail::DataPtr (*)(size_t bytes);
using fill_fn = void (*)(void* ptr, size_t n, Scalar value, DataType t);
using resize_fn = detail::DataPtr (*)(const detail::DataPtr& old, size_t old_bytes,
                                      size_t new_bytes);
using add_inplace_fn = void (*)(void* dst, const void* src, size_t n, DataType t);

LMP_DECLARE_DISPATCH(copy_fn, copy_stub)
LMP_DECLARE_DISPATCH(empty_fn, empty_stub)
LMP_DECLARE_DISPATCH(fill_fn, fill_stub)
LMP_DECLARE_DISPATCH(resize_fn, resize_stub)
LMP_DECLARE_DISPATCH(add_inplace_fn, add_inplace_stub)
}  // namespace ops

class Storage {
 public:
  Storage(size_t byte_size, DeviceType device);
  void* data() const noexcept;
  size_t byte_size() const noexcept;
  DeviceType device() const noexcept;
  void resize(size_t new_bytes);
  bool same_as(const Storage& o) const { return impl_ == o.impl_; }

 private:
  struct Impl;
  std::shared_ptr<Impl> impl_;
};

class TensorImpl {
 public:
  // Host data of any element type, converted to `dtype` on the way to
  // `device` (tensor_impl.hpp:35-53).
  template <typename T>
  TensorImpl(const std::vector<T>& data, const std::vector<size_t>& shape,
             DeviceType device, DataType dtype)
      : TensorImpl(static_cast<const void*>(data.data()), data.size(),
                   TypeOf<T>::value, shape, device, dtype) {}
  TensorImpl(const void* host, size_t count, DataType host_type,
             const std::vector<size_t>& shape, DeviceType device, DataType dtype);
  TensorImpl(Storage storage, const std::vector<size_t>& shape, DataType dtype);

  // Realises a pending lazy op first (tensor_impl.cpp:33-36).
  void* data();
  DataType type() const noexcept { return type_; }
  DeviceType device() const noexcept { return storage_.device(); }
  const std::vector<size_t>& shape() const noexcept { return shape_; }
  const std::vector<stride_t>& strides() const noexcept { return strides_; }
  size_t numel() const noexcept { return numel_; }
  size_t nbytes() const noexcept { return numel_ * dtype_size(type_); }
  bool is_deferred() const noexcept { return lazy_ != nullptr; }
  const std::shared_ptr<lazy::LazyFunction>& lazy_op() const noexcept { return lazy_; }
  void set_realized(Storage storage);
  void set_deferred(std::shared_ptr<lazy::LazyFunction> op);
  // Replaces a pending constant (a node without inputs) by another pending op
  // of the same shape and dtype, keeping this tensor's identity (a gradient
  // accumulated while still a constant).
  void replace_pending_constant(std::shared_ptr<lazy::LazyFunction> op);
  Storage storage() const noexcept { return storage_; }
  // Raw pointer without realisation; only valid for realised tensors.
  void* raw() const noexcept { return storage_.data(); }

  TensorImpl reshape(std::vector<size_t> new_shape);
  TensorImpl squeeze(size_t dim);
  TensorImpl expand_dims(size_t dim);
  Scalar index(const std::vector<size_t>& idx);

  void copy(TensorImpl& other);
  void fill(Scalar value);
  void print(std::ostream& os);

 private:
  void compute_strides();

  Storage storage_;
  std::vector<size_t> shape_;
  std::vector<stride_t> strides_;
  DataType type_;
  size_t numel_;
  std::shared_ptr<lazy::LazyFunction> lazy_;
};

class Tensor;
namespace detail {
struct UnsafeTensorAccessor;
}

class Tensor {
 public:
  Tensor() = default;
  template <typename T>
  Tensor(const std::vector<T>& data, const std::vector<size_t>& shape,
         DeviceType device = DEFAULT_DEVICE, DataType dtype = DEFAULT_DTYPE)
      : impl_(std::make_shared<TensorImpl>(data, shape, device, dtype)) {}

  bool defined() const { return impl_ != nullptr; }
  void* data();
  DataType type() const noexcept { return impl_->type(); }
  DeviceType device() const noexcept { return impl_->device(); }
  const std::vector<size_t>& shape() const noexcept { return impl_->shape(); }
  const std::vector<stride_t>& strides() const noexcept { return impl_->strides(); }
  size_t numel() const noexcept { return impl_->numel(); }

  // Copy to host and convert (tensor.hpp:54-68).
  template <typename T>
  std::vector<T> to_vector() const {
    std::vector<T> out(impl_->numel());
    if (out.empty()) return out;
    void* src = impl_->data();
    ops::copy_stub()(device(), DeviceType::CPU, src, out.data(), out.size(),
                     type(), TypeOf<T>::value);
    return out;
  }
  void copy_to_host(void* dst, DataType dst_type) const;

  Scalar index(const std::vector<size_t>& idx) const { return impl_->index(idx); }
  Tensor reshape(std::vector<size_t> new_shape) const;
  Tensor squeeze(size_t dim) const;
  Tensor expand_dims(size_t dim) const;
  Tensor to(DeviceType device) const;
  void copy(const Tensor& other);
  void fill(Scalar value);
  void realize();

  friend std::ostream& operator<<(std::ostream& os, const Tensor& t);
  friend struct detail::UnsafeTensorAccessor;

 private:
  explicit Tensor(std::shared_ptr<TensorImpl> p) : impl_(std::move(p)) {}
  std::shared_ptr<TensorImpl> impl_;
};

namespace detail {
struct UnsafeTensorAccessor {
  static const std::shared_ptr<TensorImpl>& getImpl(const Tensor& t) { return t.impl_; }
  static Tensor fromImpl(std::shared_ptr<TensorImpl> p) { return Tensor(std::move(p)); }
};
}  // namespace detail

// fill_like.hpp:13-19
Tensor full_like(const Tensor& t, Scalar value);
Tensor ones_like(const Tensor& t);
Tensor zeros_like(const Tensor& t);
// An uninitialised tensor of the given shape on `device`.
Tensor empty(const std::vector<size_t>& shape, DeviceType device, DataType dtype);

size_t shape_numel(const std::vector<size_t>& shape);

}  // namespace lmp::tensor
