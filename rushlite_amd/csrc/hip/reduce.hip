// Keep-dims reductions over the middle axis of a contiguous [outer, len,
// inner] view (Lamp3: cpu/reduct.cpp:7-49 for the semantics, reduct.cu:213-260
// for the CUDA dispatcher this replaces).
//
// Row case (inner == 1, e.g. sum/max over dim 1 of [16384,16384]):
//   long fp32 rows  -> one 256-thread workgroup per row segment, 128-bit
//                      loads, 16 independent accumulators per lane, wave64
//                      butterfly (DPP lane swaps) then LDS across the 4 waves;
//                      a row is split over several workgroups only when
//                      there are too few rows to fill 256 CUs, and the
//                      partials are folded by a second pass in fixed order.
//   short rows      -> one wave per row (softmax/loss rows like [512,1000]),
//                      float4 loads when rows are 16-byte multiples, four
//                      loads in flight per lane.
// Column case (inner > 1, e.g. sum over dim 0, the bias-gradient reduction):
//   each lane owns four adjacent columns (one float4); the four waves of a
//   workgroup share a 256-column strip and take every fourth row of a chunk
//   of the reduced axis (8 loads in flight per lane), then combine in LDS in
//   fixed wave order.  The axis is cut into S chunks so the grid holds about
//   four workgroups per CU; chunk partials [outer, S, inner] are folded by a
//   second pass, S float4 loads per lane issued together.  An axis of at
//   most 4096 rows that would need chunks (bias gradients: [batch, out] with
//   a batch of a few hundred) is reduced in one pass instead: a workgroup
//   owns a narrow strip of float4 columns and every row, its lanes split into
//   row groups that combine in LDS, so there is no second launch.  No
//   atomics: results are deterministic.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "common.hpp"
#include "ops.hpp"

namespace lmp_hip {

typedef float v4f __attribute__((ext_vector_type(4)));

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

#define LMP_WAVE_SWAP_SRC(...) __VA_ARGS__
#include "wave_swap.inc"
#undef LMP_WAVE_SWAP_SRC

// Butterfly over the 64 lanes in the order 1, 2, 4, 8, 16, 32; lane 0 holds
// the result.
template <int OP, typename T>
__device__ __forceinline__ T wave_reduce(T v) {
  using R = Reducer<OP, T>;
  v = R::combine(v, lmp_swap<1>(v));
  v = R::combine(v, lmp_swap<2>(v));
  v = R::combine(v, lmp_swap<4>(v));
  v = R::combine(v, lmp_swap<8>(v));
  v = R::combine(v, lmp_swap<16>(v));
  v = R::combine(v, lmp_swap<32>(v));
  return v;
}

template <int OP>
__device__ __forceinline__ v4f combine4(v4f a, v4f b) {
  v4f r;
  r.x = Reducer<OP, float>::combine(a.x, b.x);
  r.y = Reducer<OP, float>::combine(a.y, b.y);
  r.z = Reducer<OP, float>::combine(a.z, b.z);
  r.w = Reducer<OP, float>::combine(a.w, b.w);
  return r;
}

// Inputs of kStreamBytes or more are read with the nontemporal hint.
template <bool NT>
__device__ __forceinline__ v4f load4(const v4f* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// Block (row, part) reduces float4 [part*seg4, min(len4, (part+1)*seg4)) of
// its row and writes one value to out[row * parts + part].
template <int OP, bool NT>
__global__ __launch_bounds__(kBlock) void row_reduce_f32(
    float* __restrict__ out, const float* __restrict__ in, uint32_t len4,
    uint32_t seg4, FastDiv parts) {
  using R = Reducer<OP, float>;
  const uint32_t row = parts.div(blockIdx.x);
  const uint32_t part = blockIdx.x - row * parts.d;
  const v4f* src = reinterpret_cast<const v4f*>(in) + uint64_t(row) * len4;
  const uint32_t beg = part * seg4;
  const uint32_t end = min(len4, beg + seg4);
  const v4f id = v4f(R::identity());
  v4f acc0 = id, acc1 = id, acc2 = id, acc3 = id;
  uint32_t i = beg + threadIdx.x;
  for (; i + 3 * kBlock < end; i += 4 * kBlock) {
    v4f x0 = load4<NT>(src + i), x1 = load4<NT>(src + i + kBlock),
        x2 = load4<NT>(src + i + 2 * kBlock), x3 = load4<NT>(src + i + 3 * kBlock);
    acc0 = combine4<OP>(acc0, x0);
    acc1 = combine4<OP>(acc1, x1);
    acc2 = combine4<OP>(acc2, x2);
    acc3 = combine4<OP>(acc3, x3);
  }
  for (; i < end; i += kBlock) acc0 = combine4<OP>(acc0, load4<NT>(src + i));
  v4f acc = combine4<OP>(combine4<OP>(acc0, acc1), combine4<OP>(acc2, acc3));
  float v = R::combine(R::combine(acc.x, acc.y), R::combine(acc.z, acc.w));
  v = wave_reduce<OP, float>(v);
  __shared__ float lds[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = lds[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) r = R::combine(r, lds[w]);
    out[blockIdx.x] = r;
  }
}

// One wave per row, any dtype, any length.  Four loads per lane are issued
// before they are combined (four accumulators), so a short row costs one
// memory latency rather than one per 64 elements.
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void row_reduce_wave(
    T* __restrict__ out, const T* __restrict__ in, uint64_t rows,
    uint64_t len) {
  using R = Reducer<OP, T>;
  const uint64_t row = uint64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const T* src = in + row * len;
  T a0 = R::identity(), a1 = a0, a2 = a0, a3 = a0;
  uint64_t j = lane;
  for (; j + 192 < len; j += 256) {
    const T x0 = src[j], x1 = src[j + 64], x2 = src[j + 128], x3 = src[j + 192];
    a0 = R::combine(a0, x0);
    a1 = R::combine(a1, x1);
    a2 = R::combine(a2, x2);
    a3 = R::combine(a3, x3);
  }
  // At most three elements per lane remain (j + 192 >= len): their loads go
  // out together, then a0 takes them in index order as a loop would.
  {
    const bool t0 = j < len, t1 = j + 64 < len, t2 = j + 128 < len;
    T y0 = a0, y1 = a0, y2 = a0;
    if (t0) y0 = src[j];
    if (t1) y1 = src[j + 64];
    if (t2) y2 = src[j + 128];
    if (t0) a0 = R::combine(a0, y0);
    if (t1) a0 = R::combine(a0, y1);
    if (t2) a0 = R::combine(a0, y2);
  }
  T acc = R::combine(R::combine(a0, a1), R::combine(a2, a3));
  acc = wave_reduce<OP, T>(acc);
  if (lane == 0) out[row] = acc;
}

// One wave per fp32 row with 16-byte rows (len % 4 == 0): float4 loads, four
// in flight per lane.
template <int OP>
__global__ __launch_bounds__(kBlock) void row_reduce_wave_f32(
    float* __restrict__ out, const float* __restrict__ in, uint64_t rows,
    uint32_t len4) {
  using R = Reducer<OP, float>;
  const uint64_t row = uint64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint32_t lane = threadIdx.x & 63;
  const v4f* src = reinterpret_cast<const v4f*>(in) + row * len4;
  const v4f id = v4f(R::identity());
  v4f a0 = id, a1 = id, a2 = id, a3 = id;
  uint32_t j = lane;
  for (; j + 192 < len4; j += 256) {
    const v4f x0 = src[j], x1 = src[j + 64], x2 = src[j + 128], x3 = src[j + 192];
    a0 = combine4<OP>(a0, x0);
    a1 = combine4<OP>(a1, x1);
    a2 = combine4<OP>(a2, x2);
    a3 = combine4<OP>(a3, x3);
  }
  // At most three float4 per lane remain (j + 192 >= len4): their loads go
  // out together, then a0 takes them in index order as a loop would.
  {
    const bool t0 = j < len4, t1 = j + 64 < len4, t2 = j + 128 < len4;
    v4f y0 = id, y1 = id, y2 = id;
    if (t0) y0 = src[j];
    if (t1) y1 = src[j + 64];
    if (t2) y2 = src[j + 128];
    if (t0) a0 = combine4<OP>(a0, y0);
    if (t1) a0 = combine4<OP>(a0, y1);
    if (t2) a0 = combine4<OP>(a0, y2);
  }
  const v4f a = combine4<OP>(combine4<OP>(a0, a1), combine4<OP>(a2, a3));
  float v = R::combine(R::combine(a.x, a.y), R::combine(a.z, a.w));
  v = wave_reduce<OP, float>(v);
  if (lane == 0) out[row] = v;
}

// Fold `parts` consecutive partials per output in order.
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void fold_parts(T* __restrict__ out,
                                                     const T* __restrict__ part,
                                                     uint64_t n,
                                                     uint32_t parts) {
  using R = Reducer<OP, T>;
  const uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  T acc = R::identity();
  for (uint32_t p = 0; p < parts; ++p) acc = R::combine(acc, part[i * parts + p]);
  out[i] = acc;
}

// Column reduction, fp32.  grid = (ceil(inner4/64), S, outer); lane owns
// float4 column c4 = blockIdx.x*64 + lane, wave w takes rows r0+w, r0+w+4, ...
// of chunk s = [s*chunk, min(len, (s+1)*chunk)).  dst layout [outer, S, inner]
// (S == 1 writes the final result).
constexpr int kColUnroll = 8;
template <int OP, bool NT>
__global__ __launch_bounds__(kBlock) void col_reduce_f32(
    float* __restrict__ dst, const float* __restrict__ in, uint32_t inner4,
    uint32_t len, uint32_t chunk) {
  using R = Reducer<OP, float>;
  const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t c4 = blockIdx.x * 64 + lane;
  const uint32_t s = blockIdx.y, S = gridDim.y, o = blockIdx.z;
  const uint32_t r0 = s * chunk;
  const uint32_t r1 = min(len, r0 + chunk);
  const v4f id = v4f(R::identity());
  v4f acc[kColUnroll];
#pragma unroll
  for (int u = 0; u < kColUnroll; ++u) acc[u] = id;
  if (c4 < inner4) {
    const v4f* src = reinterpret_cast<const v4f*>(in) + uint64_t(o) * len * inner4 + c4;
    uint32_t r = r0 + w;
    for (; r + 4 * (kColUnroll - 1) < r1; r += 4 * kColUnroll) {
      v4f x[kColUnroll];
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) x[u] = load4<NT>(src + uint64_t(r + 4 * u) * inner4);
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) acc[u] = combine4<OP>(acc[u], x[u]);
    }
    for (; r < r1; r += 4) acc[0] = combine4<OP>(acc[0], load4<NT>(src + uint64_t(r) * inner4));
  }
  v4f a = acc[0];
#pragma unroll
  for (int u = 1; u < kColUnroll; ++u) a = combine4<OP>(a, acc[u]);
  __shared__ v4f lds[kWaves][64];
  lds[w][lane] = a;
  __syncthreads();
  if (w == 0 && c4 < inner4) {
    v4f t = lds[0][lane];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) t = combine4<OP>(t, lds[k][lane]);
    reinterpret_cast<v4f*>(dst)[(uint64_t(o) * S + s) * inner4 + c4] = t;
  }
}

// Column reduction in one pass for a short axis.  grid = (ceil(inner4/cw),
// 1, outer), cw = 1 << cw_log2 float4 columns per workgroup; the 256/cw row
// groups take rows g, g + 256/cw, ... (eight loads in flight per lane), then
// fold in LDS by halving in fixed order.  out layout [outer, inner4].
constexpr uint32_t kStripMaxLen = 4096;
template <int OP>
__global__ __launch_bounds__(kBlock) void col_reduce_strip_f32(
    float* __restrict__ out, const float* __restrict__ in, uint32_t inner4, uint32_t len,
    uint32_t cw_log2) {
  using R = Reducer<OP, float>;
  const uint32_t t = threadIdx.x;
  const uint32_t cw = 1u << cw_log2, rg = uint32_t(kBlock) >> cw_log2;
  const uint32_t col = t & (cw - 1), g = t >> cw_log2;
  const uint32_t c4 = blockIdx.x * cw + col;
  const uint32_t o = blockIdx.z;
  const v4f id = v4f(R::identity());
  v4f acc[kColUnroll];
#pragma unroll
  for (int u = 0; u < kColUnroll; ++u) acc[u] = id;
  if (c4 < inner4) {
    const v4f* src = reinterpret_cast<const v4f*>(in) + uint64_t(o) * len * inner4 + c4;
    uint32_t r = g;
    for (; r + rg * (kColUnroll - 1) < len; r += rg * kColUnroll) {
      v4f x[kColUnroll];
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) x[u] = src[uint64_t(r + rg * u) * inner4];
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) acc[u] = combine4<OP>(acc[u], x[u]);
    }
    for (; r < len; r += rg) acc[0] = combine4<OP>(acc[0], src[uint64_t(r) * inner4]);
  }
  v4f a = acc[0];
#pragma unroll
  for (int u = 1; u < kColUnroll; ++u) a = combine4<OP>(a, acc[u]);
  __shared__ v4f lds[kBlock];
  lds[t] = a;  // row group g, column col
  for (uint32_t half = rg >> 1; half >= 1; half >>= 1) {
    __syncthreads();
    if (g < half) {
      a = combine4<OP>(a, lds[t + half * cw]);
      lds[t] = a;
    }
  }
  if (g == 0 && c4 < inner4) reinterpret_cast<v4f*>(out)[uint64_t(o) * inner4 + c4] = a;
}

// Fold S chunk partials [outer, S, inner4] -> [outer, inner4], float4 lanes,
// in chunk order with the loads of eight chunks issued before their combines.
template <int OP>
__global__ __launch_bounds__(kBlock) void fold_chunks_f32(
    float* __restrict__ out, const float* __restrict__ part, uint64_t outer,
    uint32_t inner4, uint32_t S) {
  using R = Reducer<OP, float>;
  const uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= outer * inner4) return;
  const uint64_t o = i / inner4, c = i - o * inner4;
  const v4f* src = reinterpret_cast<const v4f*>(part) + o * S * inner4 + c;
  v4f acc = v4f(R::identity());
  uint32_t s = 0;
  for (; s + 8 <= S; s += 8) {
    v4f x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = src[uint64_t(s + u) * inner4];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = combine4<OP>(acc, x[u]);
  }
  for (; s < S; ++s) acc = combine4<OP>(acc, src[uint64_t(s) * inner4]);
  reinterpret_cast<v4f*>(out)[i] = acc;
}

// Column reduction for any dtype / alignment: one lane per column.
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void col_reduce_scalar(
    T* __restrict__ dst, const T* __restrict__ in, uint64_t inner,
    uint64_t len, uint64_t chunk) {
  using R = Reducer<OP, T>;
  const uint64_t c = uint64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (c >= inner) return;
  const uint64_t s = blockIdx.y, S = gridDim.y, o = blockIdx.z;
  const uint64_t r0 = s * chunk;
  const uint64_t r1 = min(len, r0 + chunk);
  const T* src = in + (o * len + r0) * inner + c;
  // Eight loads in flight, combined in row order (the result is the
  // sequential fold, as without the batching).
  T acc = R::identity();
  uint64_t r = r0;
  for (; r + 8 <= r1; r += 8, src += 8 * inner) {
    T x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = src[u * inner];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = R::combine(acc, x[u]);
  }
  for (; r < r1; ++r, src += inner) acc = R::combine(acc, *src);
  dst[(o * S + s) * inner + c] = acc;
}

// Column reduction with one lane per output element (o, c) of [outer, inner],
// grid-striding over them: the axis is folded sequentially from the identity
// (eight loads in flight, combined in row order).  Used when outer exceeds
// the grid's z extent, where the kernels above would need one z slice per
// outer index (reduct.cu:166-182 grid-strides over any output count too).
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void col_reduce_flat(T* __restrict__ out,
                                                          const T* __restrict__ in,
                                                          uint64_t outer, uint64_t len,
                                                          uint64_t inner) {
  using R = Reducer<OP, T>;
  const uint64_t n = outer * inner;
  const uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    const uint64_t o = i / inner, c = i - o * inner;
    const T* src = in + o * len * inner + c;
    T acc = R::identity();
    uint64_t r = 0;
    for (; r + 8 <= len; r += 8, src += 8 * inner) {
      T x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = src[u * inner];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = R::combine(acc, x[u]);
    }
    for (; r < len; ++r, src += inner) acc = R::combine(acc, *src);
    out[i] = acc;
  }
}

// Fold S chunk partials [outer, S, inner] -> [outer, inner] in chunk order.
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void fold_chunks(T* __restrict__ out,
                                                      const T* __restrict__ part,
                                                      uint64_t outer,
                                                      uint64_t inner,
                                                      uint32_t S) {
  using R = Reducer<OP, T>;
  const uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= outer * inner) return;
  const uint64_t o = i / inner, c = i - o * inner;
  const T* src = part + o * S * inner + c;
  T acc = R::identity();
  for (uint32_t s = 0; s < S; ++s) acc = R::combine(acc, src[uint64_t(s) * inner]);
  out[i] = acc;
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

uint32_t blocks_for(uint64_t n) { return uint32_t((n + kBlock - 1) / kBlock); }

// The float4 row and column kernels index within a row or a column with
// 32-bit counters that run up to a few hundred past the extent (and a chunk
// start plus a chunk length): extents of 2^31 float4 (rows) or 2^31 rows
// (columns) or more take the 64-bit kernels instead.
constexpr uint64_t kMaxU32Extent = 0x7fffffffull;

template <int OP, typename T>
int reduce_rows(Runtime* rt, T* out, const T* in, uint64_t rows, uint64_t len) {
  if constexpr (std::is_same_v<T, float>) {
    if (len >= 2048 && len % 4 == 0 && aligned16(in) && len / 4 <= kMaxU32Extent) {
      const uint64_t len4 = len / 4;
      // Enough workgroups to fill the chip twice over; split long rows only
      // when rows alone cannot.
      const uint64_t target = uint64_t(rt->cu_count) * 8;
      uint64_t parts = 1;
      if (rows < target) parts = std::min<uint64_t>((target + rows - 1) / rows,
                                                    std::max<uint64_t>(1, len4 / 1024));
      const uint64_t seg4 = (len4 + parts - 1) / parts;
      parts = (len4 + seg4 - 1) / seg4;
      if (rows * parts > 0x7fffffffull)
        return fail(LMP_ERR_UNSUPPORTED, "reduce: too many rows");
      float* dst = out;
      float* tmp = nullptr;
      if (parts > 1) {
        tmp = static_cast<float*>(scratch_alloc(rows * parts * sizeof(float)));
        if (!tmp) return LMP_ERR_OOM;
        dst = tmp;
      }
      if (rows * len4 * 16 >= kStreamBytes)
        hipLaunchKernelGGL((row_reduce_f32<OP, true>), dim3(uint32_t(rows * parts)),
                           dim3(kBlock), 0, rt->stream, dst, in, uint32_t(len4),
                           uint32_t(seg4), FastDiv(uint32_t(parts)));
      else
        hipLaunchKernelGGL((row_reduce_f32<OP, false>), dim3(uint32_t(rows * parts)),
                           dim3(kBlock), 0, rt->stream, dst, in, uint32_t(len4),
                           uint32_t(seg4), FastDiv(uint32_t(parts)));
      LMP_LAUNCH_CHECK("row_reduce_f32");
      if (parts > 1) {
        hipLaunchKernelGGL((fold_parts<OP, float>), dim3(blocks_for(rows)),
                           dim3(kBlock), 0, rt->stream, out, tmp, rows,
                           uint32_t(parts));
        LMP_LAUNCH_CHECK("fold_parts");
        scratch_free(tmp);
      }
      return LMP_OK;
    }
  }
  const uint64_t blocks = (rows + kWaves - 1) / kWaves;
  if (blocks > 0x7fffffffull) return fail(LMP_ERR_UNSUPPORTED, "reduce: too many rows");
  if constexpr (std::is_same_v<T, float>) {
    if (len % 4 == 0 && aligned16(in) && len / 4 <= kMaxU32Extent) {
      hipLaunchKernelGGL((row_reduce_wave_f32<OP>), dim3(uint32_t(blocks)), dim3(kBlock), 0,
                         rt->stream, out, in, rows, uint32_t(len / 4));
      LMP_LAUNCH_CHECK("row_reduce_wave_f32");
      return LMP_OK;
    }
  }
  hipLaunchKernelGGL((row_reduce_wave<OP, T>), dim3(uint32_t(blocks)),
                     dim3(kBlock), 0, rt->stream, out, in, rows, len);
  LMP_LAUNCH_CHECK("row_reduce_wave");
  return LMP_OK;
}

template <int OP, typename T>
int reduce_cols(Runtime* rt, T* out, const T* in, uint64_t outer, uint64_t len,
                uint64_t inner) {
  const bool vec = std::is_same_v<T, float> && inner % 4 == 0 && aligned16(in) &&
                   aligned16(out) && inner / 4 <= 0x7fffffffull &&
                   len <= kMaxU32Extent;
  // Lanes per workgroup along the columns: 64 float4 lanes (4 waves share a
  // strip) on the vector path, 256 scalar lanes otherwise.
  const uint64_t lanes = vec ? inner / 4 : inner;
  const uint64_t per_wg = vec ? 64 : kBlock;
  const uint64_t gx = (lanes + per_wg - 1) / per_wg;
  if (gx > 0x7fffffffull || outer > 65535) {
    // More outer slices than the grid's z extent (or columns than its x
    // extent): one lane per output element, grid-striding.
    const uint64_t n = outer * inner;
    const uint64_t cap = uint64_t(rt->cu_count) * 64;
    const uint64_t blocks = std::min<uint64_t>((n + kBlock - 1) / kBlock, cap);
    hipLaunchKernelGGL((col_reduce_flat<OP, T>), dim3(uint32_t(blocks)), dim3(kBlock), 0,
                       rt->stream, out, in, outer, len, inner);
    LMP_LAUNCH_CHECK("col_reduce_flat");
    return LMP_OK;
  }
  // Chunk the reduced axis until the grid reaches ~4 workgroups per CU
  // (measured best for [16384,16384]: 176 us at 4/CU vs 196 us at 8/CU),
  // keeping at least 64 rows per chunk.
  const uint64_t target = uint64_t(rt->cu_count) * 4;
  uint64_t S = 1;
  const uint64_t base = gx * outer;
  if (base < target) S = std::min<uint64_t>((target + base - 1) / base,
                                            std::max<uint64_t>(1, len / 64));
  S = std::min<uint64_t>(S, 65535);
  if constexpr (std::is_same_v<T, float>) {
    if (vec && S > 1 && len <= kStripMaxLen) {
      // One pass: about 128 workgroups where the columns allow, 4..64 float4
      // columns each.
      const uint64_t inner4 = inner / 4;
      uint32_t cw_log2 = 2;
      while (cw_log2 < 6 && (inner4 >> (cw_log2 + 1)) >= 128) ++cw_log2;
      const uint64_t gx1 = (inner4 + (1u << cw_log2) - 1) >> cw_log2;
      const dim3 grid1{uint32_t(gx1), 1u, uint32_t(outer)};
      hipLaunchKernelGGL((col_reduce_strip_f32<OP>), grid1, dim3(kBlock), 0, rt->stream, out,
                         in, uint32_t(inner4), uint32_t(len), cw_log2);
      LMP_LAUNCH_CHECK("col_reduce_strip_f32");
      return LMP_OK;
    }
  }
  const uint64_t chunk = (len + S - 1) / S;
  S = (len + chunk - 1) / chunk;
  T* dst = out;
  T* tmp = nullptr;
  if (S > 1) {
    tmp = static_cast<T*>(scratch_alloc(outer * S * inner * sizeof(T)));
    if (!tmp) return LMP_ERR_OOM;
    dst = tmp;
  }
  const dim3 grid{uint32_t(gx), uint32_t(S), uint32_t(outer)};
  if constexpr (std::is_same_v<T, float>) {
    if (vec) {
      if (outer * len * inner * sizeof(float) >= kStreamBytes)
        hipLaunchKernelGGL((col_reduce_f32<OP, true>), grid, dim3(kBlock), 0, rt->stream,
                           dst, in, uint32_t(inner / 4), uint32_t(len), uint32_t(chunk));
      else
        hipLaunchKernelGGL((col_reduce_f32<OP, false>), grid, dim3(kBlock), 0, rt->stream,
                           dst, in, uint32_t(inner / 4), uint32_t(len), uint32_t(chunk));
      LMP_LAUNCH_CHECK("col_reduce_f32");
      if (S > 1) {
        const uint64_t n4 = outer * (inner / 4);
        hipLaunchKernelGGL((fold_chunks_f32<OP>), dim3(blocks_for(n4)), dim3(kBlock), 0,
                           rt->stream, out, tmp, outer, uint32_t(inner / 4), uint32_t(S));
        LMP_LAUNCH_CHECK("fold_chunks_f32");
        scratch_free(tmp);
      }
      return LMP_OK;
    }
  }
  hipLaunchKernelGGL((col_reduce_scalar<OP, T>), grid, dim3(kBlock), 0, rt->stream, dst,
                     in, inner, len, chunk);
  LMP_LAUNCH_CHECK("col_reduce_scalar");
  if (S > 1) {
    const uint64_t n = outer * inner;
    hipLaunchKernelGGL((fold_chunks<OP, T>), dim3(blocks_for(n)), dim3(kBlock), 0,
                       rt->stream, out, tmp, outer, inner, uint32_t(S));
    LMP_LAUNCH_CHECK("fold_chunks");
    scratch_free(tmp);
  }
  return LMP_OK;
}

// An empty reduced axis leaves every output at the functor's identity
// (cpu/reduct.cpp:15-19 folds nothing into it).
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void fill_identity(T* __restrict__ out, uint64_t n) {
  const uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    out[i] = Reducer<OP, T>::identity();
}

template <int OP, typename T>
int reduce_any(Runtime* rt, T* out, const T* in, uint64_t outer, uint64_t len,
               uint64_t inner) {
  if (len == 0) {
    const uint64_t n = outer * inner;
    hipLaunchKernelGGL((fill_identity<OP, T>),
                       dim3(uint32_t(std::min<uint64_t>((n + kBlock - 1) / kBlock, 65536))),
                       dim3(kBlock), 0, rt->stream, out, n);
    LMP_LAUNCH_CHECK("fill_identity");
    return LMP_OK;
  }
  return inner == 1 ? reduce_rows<OP, T>(rt, out, in, outer, len)
                    : reduce_cols<OP, T>(rt, out, in, outer, len, inner);
}

template <typename T>
int dispatch_reduce(int op, Runtime* rt, T* out, const T* in, uint64_t outer,
                    uint64_t len, uint64_t inner) {
  switch (op) {
#define LMP_CASE(OPV) \
  case OPV:           \
    return reduce_any<OPV, T>(rt, out, in, outer, len, inner);
    LMP_CASE(LMP_RED_SUM)
    LMP_CASE(LMP_RED_MAX)
    LMP_CASE(LMP_RED_MIN)
    LMP_CASE(LMP_RED_PROD)
#undef LMP_CASE
    default:
      return fail(LMP_ERR_INVALID, "lmp_k_reduce: unknown op " + std::to_string(op));
  }
}

}  // namespace
}  // namespace lmp_hip

using namespace lmp_hip;

extern "C" int lmp_k_reduce(int op, int dtype, void* out, const void* in,
                            size_t outer, size_t len, size_t inner) {
  if (outer == 0 || inner == 0) return LMP_OK;
  if (!out || (!in && len)) return fail(LMP_ERR_INVALID, "lmp_k_reduce: null buffer");
  LMP_RUNTIME_OR_FAIL(rt);
  switch (dtype) {
    case LMP_FLOAT32:
      return dispatch_reduce<float>(op, rt, static_cast<float*>(out),
                                    static_cast<const float*>(in), outer, len, inner);
    case LMP_FLOAT64:
      return dispatch_reduce<double>(op, rt, static_cast<double*>(out),
                                     static_cast<const double*>(in), outer, len, inner);
    case LMP_INT32:
      return dispatch_reduce<int32_t>(op, rt, static_cast<int32_t*>(out),
                                      static_cast<const int32_t*>(in), outer, len, inner);
    case LMP_INT64:
      return dispatch_reduce<int64_t>(op, rt, static_cast<int64_t*>(out),
                                      static_cast<const int64_t*>(in), outer, len, inner);
    case LMP_INT16:
      return dispatch_reduce<int16_t>(op, rt, static_cast<int16_t*>(out),
                                      static_cast<const int16_t*>(in), outer, len, inner);
    case LMP_BOOL:
      return dispatch_reduce<bool>(op, rt, static_cast<bool*>(out),
                                   static_cast<const bool*>(in), outer, len, inner);
    default:
      return fail(LMP_ERR_UNSUPPORTED,
                  std::string("lmp_k_reduce: dtype ") + dtype_name(dtype));
  }
}
