/*
 * lamp_cpu.c — CPU oracle for the Lamp3 HIP backend.  TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker or the timed CPU baseline; the
 * product path never calls it.
 *
 * A plain-C restatement of Lamp3's CPU backend for fp32, written from the
 * reference's semantics (csrc/src/tensor/cpu/*):
 *   - binary ops: same-shape flat loop (cpu/binary.cpp:13-19) or the
 *     broadcast loop that decomposes the flat output index with the output
 *     strides and sums index*padded-stride per input (cpu/expand.cpp:7-22,
 *     cpu/offset_util.cpp:47-63), functors cpu/kernels.hpp:22-154;
 *   - unary ops incl. clamp (cpu/unary.cpp:7-36, kernels.hpp:70-128);
 *   - reductions: per output i, start at idx = (i/outer)*inner + i%outer and
 *     fold sequentially from the identity (cpu/reduct.cpp:7-19);
 *   - matmul: i-j-k with the sum starting at 0 and accumulating in order
 *     (cpu/matrix.cpp:8-33); transpose (cpu/matrix.cpp:17-39);
 *   - fill / add_inplace (cpu/memory.cpp:16-48).
 * Each output element is independent, so the OpenMP split over outputs does
 * not change any bit of the result.
 *
 * Build flags: the parity build (liblamp_cpu.so) is strict IEEE
 * (-ffp-contract=off, no -ffast-math) so every op rounds exactly once, which
 * is what the reference's eager per-op execution specifies.  The timing
 * build (liblamp_cpu_fast.so) adds the reference's -O3 -ffast-math
 * (CMakeLists.txt:59-64) so the CPU baseline runs at the speed the
 * reference's own flags allow.  It is linked without the fast-math startup
 * code (-mno-daz-ftz), which would otherwise switch the loading process to
 * flush-to-zero for good; lcpu_set_denormal_flush() gives that mode to the
 * timed region explicitly instead.
 */
#include <float.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <xmmintrin.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* op codes match include/lmp_hip.h */
enum {
  BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV, BIN_POW, BIN_EQ, BIN_NE, BIN_GE,
  BIN_LE, BIN_GT, BIN_LT, BIN_ABS_BACKWARD, BIN_CLAMP_BACKWARD
};
enum { UN_NEG, UN_EXP, UN_LOG, UN_SQRT, UN_ABS, UN_SIN, UN_COS, UN_TAN, UN_CLAMP };
enum { RED_SUM, RED_MAX, RED_MIN, RED_PROD };

static inline float bin_f(int op, float a, float b, float lo, float hi) {
  switch (op) {
    case BIN_ADD: return a + b;
    case BIN_SUB: return a - b;
    case BIN_MUL: return a * b;
    case BIN_DIV: return a / b;
    case BIN_POW: return powf(a, b);
    case BIN_EQ: return (float)(a == b);
    case BIN_NE: return (float)(a != b);
    case BIN_GE: return (float)(a >= b);
    case BIN_LE: return (float)(a <= b);
    case BIN_GT: return (float)(a > b);
    case BIN_LT: return (float)(a < b);
    case BIN_ABS_BACKWARD: /* (input, grad) */
      if (a > 0.0f) return b;
      if (a < 0.0f) return -b;
      return 0.0f;
    default: /* BIN_CLAMP_BACKWARD: strict bounds */
      return (a > lo && a < hi) ? b : 0.0f;
  }
}

static inline float un_f(int op, float x, float lo, float hi) {
  switch (op) {
    case UN_NEG: return -x;
    case UN_EXP: return expf(x);
    case UN_LOG: return logf(x);
    case UN_SQRT: return sqrtf(x);
    case UN_ABS: return fabsf(x);
    case UN_SIN: return sinf(x);
    case UN_COS: return cosf(x);
    case UN_TAN: return tanf(x);
    default: /* UN_CLAMP */
      if (x < lo) return lo;
      if (x > hi) return hi;
      return x;
  }
}

/* Scalar bounds arrive as double (Lamp3's Scalar) and are converted to the
 * tensor dtype once, as the functor constructors do (kernels.hpp:115-118). */
static inline float to_f32(double v) { return (float)v; }

int lcpu_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Flush-to-zero (MXCSR bit 15) and denormals-are-zero (bit 6) on or off, in
 * the calling thread and in every thread of the OpenMP team: the mode a
 * -ffast-math executable starts in.  Returns the number of threads set. */
int lcpu_set_denormal_flush(int on) {
  const unsigned bits = (1u << 15) | (1u << 6);
  int n = 1;
  _mm_setcsr(on ? (_mm_getcsr() | bits) : (_mm_getcsr() & ~bits));
#ifdef _OPENMP
#pragma omp parallel
  {
    _mm_setcsr(on ? (_mm_getcsr() | bits) : (_mm_getcsr() & ~bits));
#pragma omp single
    n = omp_get_num_threads();
  }
#endif
  return n;
}

/* out has `ndim` dims of out_shape, contiguous.  sa/sb: per-dim element
 * strides of a and b aligned to the output dims, 0 where broadcast. */
void lcpu_binary_f32(int op, float* out, const float* a, const float* b,
                     int ndim, const int64_t* out_shape, const int64_t* sa,
                     const int64_t* sb, int same_shape, double p0, double p1) {
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= out_shape[d];
  const float lo = to_f32(p0), hi = to_f32(p1);
  if (same_shape) {
#pragma omp parallel for simd
    for (int64_t i = 0; i < n; ++i) out[i] = bin_f(op, a[i], b[i], lo, hi);
    return;
  }
  int64_t ostride[64];
  {
    int64_t s = 1;
    for (int d = ndim - 1; d >= 0; --d) {
      ostride[d] = s;
      s *= out_shape[d];
    }
  }
#pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) {
    int64_t rest = i, oa = 0, ob = 0;
    for (int d = 0; d < ndim; ++d) {
      const int64_t q = rest / ostride[d];
      rest = rest % ostride[d];
      oa += q * sa[d];
      ob += q * sb[d];
    }
    out[i] = bin_f(op, a[oa], b[ob], lo, hi);
  }
}

void lcpu_unary_f32(int op, float* out, const float* in, int64_t n, double p0,
                    double p1) {
  const float lo = to_f32(p0), hi = to_f32(p1);
#pragma omp parallel for simd
  for (int64_t i = 0; i < n; ++i) out[i] = un_f(op, in[i], lo, hi);
}

static inline float red_identity(int op) {
  switch (op) {
    case RED_SUM: return 0.0f;
    case RED_MAX: return -FLT_MAX; /* numeric_limits<float>::lowest() */
    case RED_MIN: return FLT_MAX;
    default: return 1.0f;
  }
}

static inline float red_f(int op, float acc, float x) {
  switch (op) {
    case RED_SUM: return acc + x;
    case RED_MAX: return acc < x ? x : acc; /* std::max(acc, x) */
    case RED_MIN: return x < acc ? x : acc; /* std::min(acc, x) */
    default: return acc * x;
  }
}

/* Keep-dims reduction of a contiguous tensor over `axis`. */
void lcpu_reduce_f32(int op, float* out, const float* in, int ndim,
                     const int64_t* shape, int axis) {
  int64_t outer = 1; /* == strides[axis] of a contiguous tensor */
  for (int d = axis + 1; d < ndim; ++d) outer *= shape[d];
  const int64_t len = shape[axis];
  const int64_t inner = outer * len;
  /* One output per position of the other axes (reduct.cpp:26 runs over
   * out().numel()): an empty axis leaves each output at the identity. */
  int64_t nout = 1;
  for (int d = 0; d < ndim; ++d)
    if (d != axis) nout *= shape[d];
  const float id = red_identity(op);
#pragma omp parallel for
  for (int64_t i = 0; i < nout; ++i) {
    const int64_t idx = (i / outer) * inner + (i % outer);
    float acc = id;
    for (int64_t j = 0; j < len; ++j) acc = red_f(op, acc, in[idx + j * outer]);
    out[i] = acc;
  }
}

void lcpu_matmul_f32(float* c, const float* a, const float* b, int64_t m,
                     int64_t n, int64_t k) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (int64_t t = 0; t < k; ++t) sum += a[i * k + t] * b[n * t + j];
      c[i * n + j] = sum;
    }
}

void lcpu_transpose_f32(float* out, const float* in, int64_t m, int64_t n) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) out[j * m + i] = in[i * n + j];
}

void lcpu_fill_f32(float* out, int64_t n, double value) {
  const float v = to_f32(value);
#pragma omp parallel for simd
  for (int64_t i = 0; i < n; ++i) out[i] = v;
}

void lcpu_add_inplace_f32(float* dst, const float* src, int64_t n) {
#pragma omp parallel for simd
  for (int64_t i = 0; i < n; ++i) dst[i] += src[i];
}
