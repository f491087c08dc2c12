// Per-element functors of the backend, one definition shared by the eager
// kernels.  The hipRTC fusion kernels spell the same expressions in source
// form (core/hip_fusion.cpp), so eager and fused results agree bit for
// bit.  Semantics follow Lamp3's CPU functors (cpu/kernels.hpp:22-174): the
// arithmetic happens in the output dtype, comparisons yield 1 or 0 in the
// output dtype, clamp returns NaN and -0.0 unchanged, and the clamp backward
// uses strict bounds.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <limits>
#include <type_traits>

#include "lmp_hip.h"

namespace lmp_hip {

// Transcendentals run in the input precision for floating types and in
// double for integers (math_acc_t, cpu/kernels.hpp:20-21).
template <typename T>
using math_t = std::conditional_t<std::is_floating_point_v<T>, T, double>;

template <typename T>
__device__ __forceinline__ T to_t(double v) {
  return static_cast<T>(v);
}

// Integer add/sub/mul/neg wrap modulo 2^bits, which is what Lamp3's CPU
// kernels produce on two's-complement hardware; computing them in an
// unsigned type of at least int's width keeps that defined (int16 operands
// would otherwise promote to int, and int32 overflow is undefined).  bool
// keeps C++'s own rules (true + true converts back to true).
template <typename T>
struct wrap_of {
  using type = T;
};
template <> struct wrap_of<int16_t> { using type = uint32_t; };
template <> struct wrap_of<int32_t> { using type = uint32_t; };
template <> struct wrap_of<int64_t> { using type = uint64_t; };
template <typename T>
using wrap_t = typename wrap_of<T>::type;

template <int OP, typename T>
__device__ __forceinline__ T binary_apply(T a, T b, T lo, T hi) {
  using W = wrap_t<T>;
  if constexpr (OP == LMP_BIN_ADD) return static_cast<T>(W(a) + W(b));
  else if constexpr (OP == LMP_BIN_SUB) return static_cast<T>(W(a) - W(b));
  else if constexpr (OP == LMP_BIN_MUL) return static_cast<T>(W(a) * W(b));
  else if constexpr (OP == LMP_BIN_DIV) {
    if constexpr (std::is_integral_v<T>) return b == T(0) ? T(0) : T(a / b);
    else return a / b;
  }
  else if constexpr (OP == LMP_BIN_POW) {
    if constexpr (std::is_floating_point_v<T>) {
      return static_cast<T>(::pow(a, b));
    } else {
      // Integers: double pow converted back (truncation).  The reference's
      // libm pow is exact whenever the result is representable, so a result
      // within 2 ulp of an integer is snapped to it before the conversion;
      // otherwise pow(3, 1) could come back as 2.9999999999999996 and
      // truncate to 2.
      const double r = ::pow(static_cast<double>(a), static_cast<double>(b));
      const double n = ::rint(r);
      const double tol = 2.0 * ::fabs(r) * 0x1p-52;
      return static_cast<T>(::fabs(r - n) <= tol ? n : r);
    }
  }
  else if constexpr (OP == LMP_BIN_EQ) return static_cast<T>(a == b);
  else if constexpr (OP == LMP_BIN_NE) return static_cast<T>(a != b);
  else if constexpr (OP == LMP_BIN_GE) return static_cast<T>(a >= b);
  else if constexpr (OP == LMP_BIN_LE) return static_cast<T>(a <= b);
  else if constexpr (OP == LMP_BIN_GT) return static_cast<T>(a > b);
  else if constexpr (OP == LMP_BIN_LT) return static_cast<T>(a < b);
  else if constexpr (OP == LMP_BIN_ABS_BACKWARD) {
    // a = input, b = incoming gradient
    if (a > T(0)) return b;
    if (a < T(0)) return static_cast<T>(-b);
    return T(0);
  } else {  // LMP_BIN_CLAMP_BACKWARD
    return (a > lo && a < hi) ? b : T(0);
  }
}

template <int OP, typename T>
__device__ __forceinline__ T unary_apply(T x, T lo, T hi) {
  using M = math_t<T>;
  if constexpr (OP == LMP_UN_NEG) return static_cast<T>(-wrap_t<T>(x));
  else if constexpr (OP == LMP_UN_EXP) return static_cast<T>(::exp(static_cast<M>(x)));
  else if constexpr (OP == LMP_UN_LOG) return static_cast<T>(::log(static_cast<M>(x)));
  else if constexpr (OP == LMP_UN_SQRT) return static_cast<T>(::sqrt(static_cast<M>(x)));
  else if constexpr (OP == LMP_UN_ABS) return static_cast<T>(::fabs(static_cast<M>(x)));
  else if constexpr (OP == LMP_UN_SIN) return static_cast<T>(::sin(static_cast<M>(x)));
  else if constexpr (OP == LMP_UN_COS) return static_cast<T>(::cos(static_cast<M>(x)));
  else if constexpr (OP == LMP_UN_TAN) return static_cast<T>(::tan(static_cast<M>(x)));
  else {  // LMP_UN_CLAMP
    if (x < lo) return lo;
    if (x > hi) return hi;
    return x;
  }
}

// Reduction combiners with Lamp3's identities (cpu/kernels.hpp:155-174):
// lowest()/max() rather than -inf/+inf, and max(acc, x) = acc < x ? x : acc
// (std::max keeps the first argument on ties and when x is NaN).
template <int OP, typename T>
struct Reducer;

template <typename T>
struct Reducer<LMP_RED_SUM, T> {
  static __device__ __forceinline__ T identity() { return T(0); }
  static __device__ __forceinline__ T combine(T acc, T x) {
    return static_cast<T>(wrap_t<T>(acc) + wrap_t<T>(x));
  }
};
template <typename T>
struct Reducer<LMP_RED_MAX, T> {
  static __device__ __forceinline__ T identity() {
    return std::numeric_limits<T>::lowest();
  }
  static __device__ __forceinline__ T combine(T acc, T x) {
    return acc < x ? x : acc;
  }
};
template <typename T>
struct Reducer<LMP_RED_MIN, T> {
  static __device__ __forceinline__ T identity() {
    return std::numeric_limits<T>::max();
  }
  static __device__ __forceinline__ T combine(T acc, T x) {
    return x < acc ? x : acc;
  }
};
template <typename T>
struct Reducer<LMP_RED_PROD, T> {
  static __device__ __forceinline__ T identity() { return T(1); }
  static __device__ __forceinline__ T combine(T acc, T x) {
    return static_cast<T>(wrap_t<T>(acc) * wrap_t<T>(x));
  }
};

}  // namespace lmp_hip
