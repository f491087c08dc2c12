// Error macros and the basic enums of the host framework.
//
// Mirrors Lamp3's conventions (common/assert.hpp:32-160): misuse of the API
// (bad shapes, devices, dtypes) throws std::runtime_error, which pybind11
// surfaces as RuntimeError; failures reported by the device backend throw the
// backend's own message the same way instead of terminating the process.
#pragma once

#include <cstddef>
#include <cstdint>
#include <ostream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "lmp_hip.h"

namespace lmp {

namespace detail {
// Collects a streamed message and throws it from the destructor of the
// temporary built by LMP_CHECK (the statement's end).
class CheckFailure {
 public:
  CheckFailure(const char* cond, const char* file, int line) {
    os_ << file << ":" << line << ": check `" << cond << "` failed: ";
  }
  template <typename T>
  CheckFailure& operator<<(const T& v) {
    os_ << v;
    return *this;
  }
  template <typename T>
  CheckFailure& operator<<(const std::vector<T>& v) {
    os_ << "[";
    for (size_t i = 0; i < v.size(); ++i) os_ << (i ? ", " : "") << v[i];
    os_ << "]";
    return *this;
  }
  [[noreturn]] void raise() const { throw std::runtime_error(os_.str()); }

 private:
  std::ostringstream os_;
};
struct Raiser {
  [[noreturn]] void operator&(const CheckFailure& f) const { f.raise(); }
};
}  // namespace detail

}  // namespace lmp

#define LMP_CHECK(cond)                      \
  if (cond) {                                \
  } else                                     \
    ::lmp::detail::Raiser() &                \
        ::lmp::detail::CheckFailure(#cond, __FILE__, __LINE__)

#define LMP_INTERNAL_ASSERT(cond) LMP_CHECK(cond) << "internal error: "

namespace lmp {

// A C-ABI status from liblmp_hip turned into an exception.
void hip_throw(int status, const char* what);
inline void hip_ok(int status, const char* what) {
  if (status != LMP_OK) hip_throw(status, what);
}

namespace tensor {

using Scalar = double;

// Codes equal lmp::tensor::DataType (data_type.hpp:25-32) and lmp_dtype.
enum class DataType : uint8_t {
  Bool = 0,
  Int16 = 1,
  Int32 = 2,
  Int64 = 3,
  Float32 = 4,
  Float64 = 5
};

// Device slots of the dispatch tables (device_type.hpp:12).  The GPU slot is
// the HIP device; CUDA is kept as an alias so code written against the
// reference's enum keeps compiling and selecting the GPU.
enum class DeviceType : size_t { CPU = 0, HIP = 1, CUDA = 1, Count = 2 };

constexpr DataType DEFAULT_DTYPE = DataType::Float32;
constexpr DeviceType DEFAULT_DEVICE = DeviceType::HIP;

// Output dtype of a binary op: the larger enum value (data_type.hpp:77-80).
inline DataType type_upcast(DataType a, DataType b) {
  return static_cast<uint8_t>(a) >= static_cast<uint8_t>(b) ? a : b;
}

inline size_t dtype_size(DataType t) {
  switch (t) {
    case DataType::Bool: return 1;
    case DataType::Int16: return 2;
    case DataType::Int32: return 4;
    case DataType::Int64: return 8;
    case DataType::Float32: return 4;
    case DataType::Float64: return 8;
  }
  return 0;
}

const char* dtype_name(DataType t);
const char* device_name(DeviceType d);
std::ostream& operator<<(std::ostream& os, DataType t);
std::ostream& operator<<(std::ostream& os, DeviceType d);

template <typename T>
struct TypeOf;
template <> struct TypeOf<bool> { static constexpr DataType value = DataType::Bool; };
template <> struct TypeOf<int16_t> { static constexpr DataType value = DataType::Int16; };
template <> struct TypeOf<int32_t> { static constexpr DataType value = DataType::Int32; };
template <> struct TypeOf<int64_t> { static constexpr DataType value = DataType::Int64; };
template <> struct TypeOf<float> { static constexpr DataType value = DataType::Float32; };
template <> struct TypeOf<double> { static constexpr DataType value = DataType::Float64; };

// Call f(T{}) with T the C++ type of `t`.
template <typename F>
decltype(auto) visit_dtype(DataType t, F&& f) {
  switch (t) {
    case DataType::Bool: return f(bool{});
    case DataType::Int16: return f(int16_t{});
    case DataType::Int32: return f(int32_t{});
    case DataType::Int64: return f(int64_t{});
    case DataType::Float32: return f(float{});
    case DataType::Float64: return f(double{});
  }
  throw std::runtime_error("unknown DataType");
}

using stride_t = int64_t;
constexpr size_t kMaxDims = LMP_MAX_DIMS;

std::ostream& operator<<(std::ostream& os, const std::vector<size_t>& v);

}  // namespace tensor
}  // namespace lmp
