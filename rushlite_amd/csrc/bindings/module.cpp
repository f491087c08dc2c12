// pybind11 module rushlite_amd._C: the Python surface of Lamp3's bindings
// (csrc/bindings/core.cpp:21-36 and the headers it includes) over this
// framework, plus two additions: Variable/_Tensor accept numpy arrays and
// expose .numpy() (bulk data without Python lists), and _stats() reports
// kernel launches and fusion-cache activity.
#include <pybind11/numpy.h>
#include <pybind11/operators.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <sstream>

#include "autograd.hpp"

namespace py = pybind11;
using lmp::autograd::Variable;
using lmp::tensor::DataType;
using lmp::tensor::DeviceType;
using lmp::tensor::Scalar;
using lmp::tensor::Tensor;
namespace ag = lmp::autograd;
namespace tops = lmp::tensor::ops;

namespace lmp::tensor::hip {
std::string fused_source_for(TensorImpl* root);
bool realize_into(TensorImpl* root, const Storage& target);
}

namespace {

// Values and shape of Python data that is not an ndarray (nested lists or
// tuples of numbers, or one number), read through numpy.asarray: numpy works
// out the shape and refuses ragged nesting, the dtype kind tells numbers from
// anything else (an object array is checked item by item), and the values
// arrive as float64 -- Lamp3's Scalar -- for
// the tensor constructor to convert to the target dtype.  The two error texts
// are the ones Lamp3's Python users see (bindings/variable.hpp:21-48).
void values_of(const py::handle& data, std::vector<Scalar>& flat, std::vector<size_t>& shape) {
  py::array arr;
  try {
    arr = py::module_::import("numpy").attr("asarray")(data);
  } catch (py::error_already_set& e) {
    if (e.matches(PyExc_ValueError)) throw py::value_error("Rushlite: array must be uniform");
    throw py::value_error("Rushlite: invalid input type");
  }
  const char kind = arr.dtype().kind();
  if (kind == 'O') {
    // Items numpy kept as Python objects: integers beyond 64 bits (Lamp3
    // casts each item to double, so they are taken at their float64 value)
    // or, on numpy before 1.24, ragged nesting.  Anything else is not a number.
    py::module_ np = py::module_::import("numpy");
    const py::object complex_kind = np.attr("complexfloating");
    shape.assign(arr.shape(), arr.shape() + arr.ndim());
    if (shape.empty()) shape.push_back(1);
    flat.clear();
    for (const py::handle item : arr.attr("ravel")()) {
      if (py::isinstance<py::list>(item) || py::isinstance<py::tuple>(item))
        throw py::value_error("Rushlite: array must be uniform");
      if (item.is_none() || py::isinstance<py::str>(item) || py::isinstance<py::bytes>(item) ||
          PyComplex_Check(item.ptr()) || py::isinstance(item, complex_kind) ||
          !PyNumber_Check(item.ptr()))
        throw py::value_error("Rushlite: invalid input type");
      const double v = PyFloat_AsDouble(item.ptr());
      if (v == -1.0 && PyErr_Occurred()) {
        PyErr_Clear();
        throw py::value_error("Rushlite: invalid input type");
      }
      flat.push_back(v);
    }
    return;
  }
  if (kind != 'b' && kind != 'i' && kind != 'u' && kind != 'f')
    throw py::value_error("Rushlite: invalid input type");
  const auto values = py::array_t<double, py::array::c_style | py::array::forcecast>::ensure(arr);
  if (!values) throw py::value_error("Rushlite: invalid input type");
  shape.assign(values.shape(), values.shape() + values.ndim());
  if (shape.empty()) shape.push_back(1);  // one number: a [1] tensor, as for a 0-d ndarray
  flat.assign(values.data(), values.data() + values.size());
}

DataType dtype_of_numpy(const py::dtype& dt) {
  if (dt.is(py::dtype::of<float>())) return DataType::Float32;
  if (dt.is(py::dtype::of<double>())) return DataType::Float64;
  if (dt.is(py::dtype::of<int32_t>())) return DataType::Int32;
  if (dt.is(py::dtype::of<int64_t>())) return DataType::Int64;
  if (dt.is(py::dtype::of<int16_t>())) return DataType::Int16;
  if (dt.is(py::dtype::of<bool>())) return DataType::Bool;
  throw py::type_error("unsupported numpy dtype");
}

py::dtype numpy_of(DataType t) {
  switch (t) {
    case DataType::Bool: return py::dtype::of<bool>();
    case DataType::Int16: return py::dtype::of<int16_t>();
    case DataType::Int32: return py::dtype::of<int32_t>();
    case DataType::Int64: return py::dtype::of<int64_t>();
    case DataType::Float32: return py::dtype::of<float>();
    case DataType::Float64: return py::dtype::of<double>();
  }
  throw py::type_error("unknown dtype");
}

Tensor tensor_from(const py::object& data, DeviceType device, DataType dtype) {
  if (py::isinstance<py::array>(data)) {
    py::array arr = py::array::ensure(data, py::array::c_style);
    if (!arr) throw py::type_error("array is not C-contiguous convertible");
    std::vector<size_t> shape(arr.shape(), arr.shape() + arr.ndim());
    if (shape.empty()) shape.push_back(1);
    auto impl = std::make_shared<lmp::tensor::TensorImpl>(
        arr.data(), static_cast<size_t>(arr.size()), dtype_of_numpy(arr.dtype()), shape,
        device, dtype);
    return lmp::tensor::detail::UnsafeTensorAccessor::fromImpl(impl);
  }
  std::vector<Scalar> flat;
  std::vector<size_t> shape;
  values_of(data, flat, shape);
  return Tensor(flat, shape, device, dtype);
}

py::array to_numpy(const Tensor& t) {
  std::vector<py::ssize_t> shape(t.shape().begin(), t.shape().end());
  py::array out(numpy_of(t.type()), shape);
  t.copy_to_host(out.mutable_data(), t.type());
  return out;
}

template <typename T>
std::string repr(const T& v) {
  std::ostringstream os;
  os << v;
  return os.str();
}

std::ostream& print_var(std::ostream& os, const Variable& v) {
  os << "Variable(requires_grad=" << (v.requires_grad() ? "true" : "false")
     << ", data=" << v.data();
  if (v.requires_grad()) os << ", grad=" << v.grad();
  else os << ", grad=0";
  os << ", grad_fn=" << (v.grad_fn_ptr() ? v.grad_fn_ptr()->name : "0") << ")";
  return os;
}

bool device_available() {
  int n = 0;
  lmp_rt_device_count(&n);
  return n > 0;
}

void device_sync() {
  if (device_available()) lmp::hip_ok(lmp_rt_synchronize(), "lmp_rt_synchronize");
}

Variable s2v(const Variable& like, Scalar s) { return ag::scalar_var(like, s); }

// One captured device graph (lmp_rt_graph_*): the library stream's work
// between begin() and end(), replayed by launch().  Scalars the capture reads
// are kept here for the graph's lifetime.
struct HipGraph {
  void* handle = nullptr;
  bool open = false;
  std::vector<Tensor> keep;

  void begin() {
    LMP_CHECK(!open && !handle) << "graph: already captured (make a new Graph)";
    lmp::hip_ok(lmp_rt_graph_begin(), "lmp_rt_graph_begin");
    open = true;
    lmp::tensor::set_graph_keep_alive(&keep);
  }
  void end() {
    LMP_CHECK(open) << "graph: no capture is open";
    lmp::tensor::set_graph_keep_alive(nullptr);
    open = false;
    lmp::hip_ok(lmp_rt_graph_end(&handle), "lmp_rt_graph_end");
  }
  void abort() {
    if (!open) return;
    lmp::tensor::set_graph_keep_alive(nullptr);
    open = false;
    lmp_rt_graph_abort();
  }
  void launch() {
    LMP_CHECK(handle) << "graph: nothing captured";
    lmp::hip_ok(lmp_rt_graph_launch(handle), "lmp_rt_graph_launch");
  }
  ~HipGraph() {
    abort();
    if (handle) lmp_rt_graph_destroy(handle);
  }
};

}  // namespace

PYBIND11_MODULE(_C, m) {
  m.doc() = "Lamp3 on AMD Instinct MI355X: HIP device backend + host framework";

  py::enum_<DataType>(m, "dtype")
      .value("float32", DataType::Float32)
      .value("float64", DataType::Float64)
      .value("bool", DataType::Bool)
      .value("int16", DataType::Int16)
      .value("int32", DataType::Int32)
      .value("int64", DataType::Int64)
      .export_values();

  py::enum_<DeviceType>(m, "device")
      .value("cpu", DeviceType::CPU)
      .value("hip", DeviceType::HIP)
      .value("cuda", DeviceType::CUDA);  // alias of hip (bindings/device_type.hpp:9-11)

  for (const char* name : {"cuda", "hip"}) {
    auto sub = m.def_submodule(name);
    sub.def("sync", &device_sync, "Wait for all queued device work.");
    sub.def("is_available", &device_available);
  }
  py::class_<HipGraph>(m.attr("hip"), "_Graph")
      .def(py::init<>())
      .def("begin", &HipGraph::begin)
      .def("end", &HipGraph::end)
      .def("abort", &HipGraph::abort)
      .def("launch", &HipGraph::launch)
      .def_property_readonly("captured", [](const HipGraph& g) { return g.handle != nullptr; })
      .def_property_readonly("capturing", [](const HipGraph& g) { return g.open; });
  m.attr("hip").attr("device_info") = py::cpp_function([]() {
    lmp_rt_info info{};
    lmp::hip_ok(lmp_rt_device_info(&info), "lmp_rt_device_info");
    py::dict d;
    d["name"] = std::string(info.name);
    d["arch"] = std::string(info.arch);
    d["cu_count"] = info.cu_count;
    d["wave_size"] = info.wave_size;
    d["lds_bytes_per_cu"] = info.lds_bytes_per_cu;
    d["total_mem_bytes"] = info.total_mem_bytes;
    d["clock_khz"] = info.clock_khz;
    return d;
  });

  // ----------------------------------------------------------------- _Tensor
  auto tcls = py::class_<Tensor>(m, "_Tensor")
      .def(py::init([](const py::object& data, const std::vector<size_t>& shape,
                       DeviceType device, DataType dtype) {
             Tensor t = tensor_from(data, device, dtype);
             if (!shape.empty() && shape != t.shape()) t = t.reshape(shape);
             return t;
           }),
           py::arg("data"), py::arg("shape"), py::arg("device"), py::arg("dtype"))
      .def_property_readonly("shape", &Tensor::shape)
      .def_property_readonly("device", &Tensor::device)
      .def_property_readonly("dtype", &Tensor::type)
      .def("index", &Tensor::index, py::arg("idx"))
      .def("reshape", &Tensor::reshape, py::arg("new_shape"))
      .def("squeeze", &Tensor::squeeze, py::arg("dim"))
      .def("expand_dims", &Tensor::expand_dims, py::arg("dim"))
      .def("to", &Tensor::to, py::arg("device"))
      .def("copy", &Tensor::copy, py::arg("other"))
      .def("fill", &Tensor::fill, py::arg("item"))
      .def("realize", &Tensor::realize)
      .def("tolist", [](const Tensor& t) { return t.to_vector<double>(); })
      .def("numpy", &to_numpy)
      .def("__repr__", &repr<Tensor>);
#define LMP_TENSOR_OP(op)                        \
  tcls.def(py::self op py::self)                 \
      .def(py::self op Scalar())                 \
      .def(Scalar() op py::self);
  LMP_TENSOR_OP(+)
  LMP_TENSOR_OP(-)
  LMP_TENSOR_OP(*)
  LMP_TENSOR_OP(/)
  LMP_TENSOR_OP(==)
  LMP_TENSOR_OP(!=)
  LMP_TENSOR_OP(<)
  LMP_TENSOR_OP(<=)
  LMP_TENSOR_OP(>)
  LMP_TENSOR_OP(>=)
#undef LMP_TENSOR_OP
  tcls.def(-py::self);

  // ---------------------------------------------------------------- Variable
  auto vcls = py::class_<Variable>(m, "Variable")
      .def(py::init<Tensor, bool>(), py::arg("data"), py::arg("requires_grad") = false)
      .def(py::init([](const py::object& data, bool requires_grad, DeviceType device,
                       DataType dtype) {
             return Variable(tensor_from(data, device, dtype), requires_grad);
           }),
           py::arg("data"), py::arg("requires_grad") = false,
           py::arg("device") = lmp::tensor::DEFAULT_DEVICE,
           py::arg("dtype") = lmp::tensor::DEFAULT_DTYPE)
      .def_property_readonly("data", &Variable::data)
      .def_property_readonly("grad", &Variable::grad)
      .def_property_readonly("grad_fn",
                             [](const Variable& v) -> py::object {
                               if (!v.grad_fn_ptr()) return py::none();
                               return py::str(v.grad_fn_ptr()->name);
                             })
      .def_property_readonly("requires_grad", &Variable::requires_grad)
      .def_property_readonly("shape", [](const Variable& v) { return v.data().shape(); })
      .def_property_readonly("device", [](const Variable& v) { return v.data().device(); })
      .def_property_readonly("dtype", [](const Variable& v) { return v.data().type(); })
      .def_property_readonly("ndim",
                             [](const Variable& v) { return v.data().shape().size(); })
      .def("backward", &Variable::backward)
      .def("tolist", [](const Variable& v) { return v.data().to_vector<double>(); })
      .def("numpy", [](const Variable& v) { return to_numpy(v.data()); })
      .def("zero_grad", &Variable::zero_grad)
      .def("realize", &Variable::realize)
      .def("__repr__", [](const Variable& v) {
        std::ostringstream os;
        print_var(os, v);
        return os.str();
      });
#define LMP_VAR_OP(op)                           \
  vcls.def(py::self op py::self)                 \
      .def(py::self op Scalar())                 \
      .def(Scalar() op py::self);
  LMP_VAR_OP(+)
  LMP_VAR_OP(-)
  LMP_VAR_OP(*)
  LMP_VAR_OP(/)
  LMP_VAR_OP(==)
  LMP_VAR_OP(!=)
  LMP_VAR_OP(<)
  LMP_VAR_OP(<=)
  LMP_VAR_OP(>)
  LMP_VAR_OP(>=)
#undef LMP_VAR_OP
  vcls.def(-py::self)
      .def("__abs__", &ag::ops::abs, py::is_operator())
      .def("__matmul__", &ag::ops::matmul, py::is_operator())
      .def("__pow__", &ag::ops::pow, py::is_operator())
      .def("__pow__", [](const Variable& a, Scalar s) { return ag::ops::pow(a, s2v(a, s)); },
           py::is_operator())
      .def("__rpow__", [](const Variable& a, Scalar s) { return ag::ops::pow(s2v(a, s), a); },
           py::is_operator())
      .def("exp", &ag::ops::exp)
      .def("log", &ag::ops::log)
      .def("sqrt", &ag::ops::sqrt)
      .def("abs", &ag::ops::abs)
      .def("sin", &ag::ops::sin)
      .def("cos", &ag::ops::cos)
      .def("tan", &ag::ops::tan)
      .def("to", &ag::ops::to, py::arg("device"))
      .def("reshape", &ag::ops::reshape, py::arg("shape"))
      .def("squeeze", &ag::ops::squeeze, py::arg("axis"))
      .def("expand_dims", &ag::ops::expand_dims, py::arg("axis"))
      .def("clamp", &ag::ops::clamp, py::arg("min"), py::arg("max"))
      .def("sum", &ag::ops::sum, py::arg("axis"))
      .def("max", &ag::ops::max, py::arg("axis"))
      .def("min", &ag::ops::min, py::arg("axis"))
      .def("prod", &ag::ops::prod, py::arg("axis"))
      .def("matmul", &ag::ops::matmul, py::arg("other"))
      .def("transpose", &ag::ops::transpose)
      .def_property_readonly("T", &ag::ops::transpose);

  // ------------------------------------------------------------ functions
#define LMP_BIND_BINARY(name)                                                   \
  m.def(#name, &ag::ops::name, py::arg("a"), py::arg("b"));                     \
  m.def(#name, [](const Variable& a, Scalar b) { return ag::ops::name(a, s2v(a, b)); }, \
        py::arg("a"), py::arg("b"));                                            \
  m.def(#name, [](Scalar a, const Variable& b) { return ag::ops::name(s2v(b, a), b); }, \
        py::arg("a"), py::arg("b"));
  LMP_BIND_BINARY(add)
  LMP_BIND_BINARY(sub)
  LMP_BIND_BINARY(mul)
  LMP_BIND_BINARY(div)
  LMP_BIND_BINARY(pow)
  LMP_BIND_BINARY(eq)
  LMP_BIND_BINARY(ne)
  LMP_BIND_BINARY(ge)
  LMP_BIND_BINARY(le)
  LMP_BIND_BINARY(gt)
  LMP_BIND_BINARY(lt)
#undef LMP_BIND_BINARY
  for (auto [name, fn] : std::vector<std::pair<const char*, Variable (*)(const Variable&)>>{
           {"neg", &ag::ops::neg}, {"exp", &ag::ops::exp}, {"log", &ag::ops::log},
           {"sqrt", &ag::ops::sqrt}, {"abs", &ag::ops::abs}, {"sin", &ag::ops::sin},
           {"cos", &ag::ops::cos}, {"tan", &ag::ops::tan}, {"transpose", &ag::ops::transpose}})
    m.def(name, fn, py::arg("a"));
  m.def("clamp", &ag::ops::clamp, py::arg("a"), py::arg("min"), py::arg("max"));
  m.def("matmul", &ag::ops::matmul, py::arg("a"), py::arg("b"));
  m.def("linear", &ag::ops::linear, py::arg("x"), py::arg("w"), py::arg("b"),
        "x @ w + b in one GEMM (the bias added in its epilogue); the same values as "
        "matmul followed by the broadcast add.");
  m.def("linear_relu", &ag::ops::linear_relu, py::arg("x"), py::arg("w"), py::arg("b"),
        "clamp(x @ w + b, 0, DBL_MAX) (Linear then ReLU) as one node: on the HIP device one "
        "GEMM whose epilogue adds the bias and applies ReLU; the same values and gradients "
        "as the two layers.");
  m.def("sum", &ag::ops::sum, py::arg("a"), py::arg("axis"));
  m.def("max", &ag::ops::max, py::arg("a"), py::arg("axis"));
  m.def("min", &ag::ops::min, py::arg("a"), py::arg("axis"));
  m.def("prod", &ag::ops::prod, py::arg("a"), py::arg("axis"));
  m.def("reshape", &ag::ops::reshape, py::arg("a"), py::arg("shape"));
  m.def("squeeze", &ag::ops::squeeze, py::arg("a"), py::arg("axis"));
  m.def("expand_dims", &ag::ops::expand_dims, py::arg("a"), py::arg("axis"));
  m.def("to", &ag::ops::to, py::arg("a"), py::arg("device"));

  m.def("zeros", &ag::zeros, py::arg("shape"), py::arg("requires_grad") = false,
        py::arg("device") = lmp::tensor::DEFAULT_DEVICE,
        py::arg("dtype") = lmp::tensor::DEFAULT_DTYPE);
  m.def("ones", &ag::ones, py::arg("shape"), py::arg("requires_grad") = false,
        py::arg("device") = lmp::tensor::DEFAULT_DEVICE,
        py::arg("dtype") = lmp::tensor::DEFAULT_DTYPE);
  m.def("rand", &ag::rand, py::arg("shape"), py::arg("requires_grad") = false,
        py::arg("device") = lmp::tensor::DEFAULT_DEVICE,
        py::arg("dtype") = lmp::tensor::DEFAULT_DTYPE);
  m.def("randn", &ag::randn, py::arg("mean"), py::arg("var"), py::arg("shape"),
        py::arg("requires_grad") = false, py::arg("device") = lmp::tensor::DEFAULT_DEVICE,
        py::arg("dtype") = lmp::tensor::DEFAULT_DTYPE);
  m.def("manual_seed", &ag::manual_seed, py::arg("seed"));

  m.def("set_capture_enabled", &lmp::tensor::lazy::set_capture_enabled);
  m.def("is_capture_enabled", &lmp::tensor::lazy::is_capture_enabled);
  m.def("set_grad_enabled", &ag::set_grad_enabled);
  m.def("is_grad_enabled", &ag::is_grad_enabled);

  m.def("_stats", []() {
    const auto& s = lmp::tensor::backend_stats();
    py::dict d;
    d["eager_launches"] = s.eager_launches;
    d["fused_launches"] = s.fused_launches;
    d["fused_nodes"] = s.fused_nodes;
    d["jit_compiles"] = s.jit_compiles;
    d["jit_cache_hits"] = s.jit_cache_hits;
    d["fused_host_ns"] = s.fused_host_ns;
    d["gemm_host_ns"] = s.gemm_host_ns;
    uint64_t kernels = 0;
    if (lmp_rt_kernel_launch_count(&kernels) == LMP_OK) d["kernels"] = kernels;
    lmp_rt_pool_stats ps{};
    if (lmp_rt_pool_stats_get(&ps) == LMP_OK) {
      d["pool_reserved_bytes"] = ps.reserved_bytes;
      d["pool_allocated_bytes"] = ps.allocated_bytes;
      d["pool_device_mallocs"] = ps.device_mallocs;
    }
    return d;
  });
  m.def("_fused_source", [](const Variable& v) {
    auto impl = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(v.data());
    return lmp::tensor::hip::fused_source_for(impl.get());
  });
  m.def("_is_deferred", [](const Variable& v) {
    return lmp::tensor::detail::UnsafeTensorAccessor::getImpl(v.data())->is_deferred();
  });
  // dst receives src's value.  A pending fused elementwise src is computed
  // straight into dst's buffer and then shares it (True); anything else is
  // realised and copied (False).
  m.def("_realize_into", [](Tensor& dst, Tensor& src) {
    auto di = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(dst);
    auto si = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(src);
    LMP_CHECK(di->numel() == si->numel() && di->type() == si->type() &&
              di->device() == si->device())
        << "realize_into: tensors differ in size, dtype or device";
    dst.realize();
    if (si->device() == DeviceType::HIP &&
        lmp::tensor::hip::realize_into(si.get(), di->storage()))
      return true;
    dst.copy(src);
    return false;
  });
  // Realises every pending tensor of `items` (Variables or tensors) together:
  // on the HIP device their elementwise regions (an optimizer's per-parameter
  // updates) run as one kernel where they are independent.
  m.def("realize_all", [](const py::iterable& items) {
    std::vector<Tensor> keep;
    std::vector<lmp::tensor::TensorImpl*> roots;
    for (const py::handle& h : items) {
      Tensor t = py::isinstance<Variable>(h) ? h.cast<Variable>().data() : h.cast<Tensor>();
      auto impl = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(t);
      if (!impl->is_deferred()) continue;
      roots.push_back(impl.get());
      keep.push_back(t);
    }
    lmp::tensor::lazy::realize_many(roots, {});
  });
  // _realize_into for many pairs at once (one grouped kernel for the pending
  // elementwise sources that can be computed in place); returns, per pair,
  // whether src now shares dst's buffer.
  m.def("_realize_into_many", [](std::vector<Tensor> dsts, std::vector<Tensor> srcs) {
    LMP_CHECK(dsts.size() == srcs.size()) << "realize_into: one source per destination";
    std::vector<lmp::tensor::TensorImpl*> roots;
    std::vector<lmp::tensor::Storage> stores;
    stores.reserve(dsts.size());
    for (size_t i = 0; i < dsts.size(); ++i) {
      auto di = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(dsts[i]);
      auto si = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(srcs[i]);
      LMP_CHECK(di->numel() == si->numel() && di->type() == si->type() &&
                di->device() == si->device())
          << "realize_into: tensors differ in size, dtype or device";
      dsts[i].realize();
      stores.push_back(di->storage());
    }
    std::vector<const lmp::tensor::Storage*> targets;
    for (size_t i = 0; i < srcs.size(); ++i) {
      auto si = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(srcs[i]);
      if (!si->is_deferred() || si->device() != DeviceType::HIP) continue;
      roots.push_back(si.get());
      targets.push_back(&stores[i]);
    }
    if (!roots.empty()) lmp::tensor::lazy::realize_many(roots, targets);
    std::vector<bool> shared;
    for (size_t i = 0; i < srcs.size(); ++i) {
      auto si = lmp::tensor::detail::UnsafeTensorAccessor::getImpl(srcs[i]);
      const bool same = si->raw() == stores[i].data();
      if (!same) dsts[i].copy(srcs[i]);
      shared.push_back(same);
    }
    return shared;
  });
  m.def("_storage_ptr", [](const Tensor& t) {
    return reinterpret_cast<uintptr_t>(
        lmp::tensor::detail::UnsafeTensorAccessor::getImpl(t)->raw());
  });
}
