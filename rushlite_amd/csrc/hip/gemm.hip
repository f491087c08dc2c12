// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32) and transpose.
//
// C[m,n] (+)= sum_k opA(A)[m,k] * opB(B)[k,n], row-major, any of the four
// operand orientations, so Linear's backward (dY*W^T and X^T*dY) needs no
// materialised transpose (the reference transposes then multiplies,
// functions/matrix_ops.cpp:8-24, with a SIMT kernel, matrix.cu:21-145).
//
// Tiling.  A workgroup of 4 waves owns a BM x BN tile of C; the waves form a
// WGM x WGN grid and each wave owns TM x TN blocks of 32x32, accumulated by
// one MFMA chain per block.  K advances BK = 32 at a time through two LDS
// buffers with one barrier per K step.  gemm_f32_mfma stages the next tile's
// global loads in registers and writes them to the other LDS buffer after the
// current tile's MFMAs; gemm_f32_lds (operands that allow 128-bit loads;
// 128 x 128, 256 x 128 and 256 x 256 tiles) loads straight into LDS and
// pipelines its fragment reads inside the tile.
//
// MFMA operand layout.  For 32x32x2 a lane l supplies A[i][kk] and B[kk][j]
// with i = j = l % 32 and kk = l / 32.  Within a BK tile, MFMA step s pairs
// k = s (lanes 0-31) with k = s + BK/2 (lanes 32-63), so a lane's 16 A values
// (and B values) for one tile are contiguous in k: a row-major-in-k LDS tile
// is read with four 128-bit LDS loads per 32-row block.  Sum order over k is a
// permutation of the serial order, which the 1e-4 tolerance admits.
// Accumulator layout: register r of a lane holds row 8*(r/4) + 4*(l/32) + r%4,
// column l % 32.
//
// Grid.  Workgroup ids are first regrouped so each of the 8 XCDs (which
// receive ids round-robin) processes a contiguous run of tiles, then tiles
// are walked in groups of 8 tile-rows so neighbours share A and B panels in
// that XCD's L2.  When the tile count cannot fill the chip, K is split over
// blockIdx.z into fp32 partials folded in split order by a second kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <limits>
#include <string>
#include <type_traits>

#include "common.hpp"

namespace lmp_hip {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

namespace {

constexpr int kThreads = 256;
constexpr int kBK = 32;
constexpr int kPad = 4;

template <int WGM_, int WGN_, int TM_, int TN_>
struct Cfg {
  static constexpr int WGM = WGM_, WGN = WGN_, TM = TM_, TN = TN_;
  static constexpr int BM = WGM * TM * 32;
  static constexpr int BN = WGN * TN * 32;
  static_assert(WGM * WGN == 4, "four waves per workgroup");
};

using CfgLarge = Cfg<2, 2, 2, 2>;   // 128 x 128
using CfgMid = Cfg<2, 2, 1, 2>;     // 64 x 128
using CfgSmall = Cfg<2, 2, 1, 1>;   // 64 x 64
using CfgSkinny = Cfg<1, 4, 1, 2>;  // 32 x 256

template <class C, bool TA>
constexpr int a_lds_floats() {
  return TA ? kBK * (C::BM + kPad) : C::BM * (kBK + kPad);
}
template <class C, bool TB>
constexpr int b_lds_floats() {
  return TB ? C::BN * (kBK + kPad) : kBK * (C::BN + kPad);
}

struct GemmArgs {
  const float* a;
  const float* b;
  float* c;        // final output (split == 1) or partial buffer base
  int m, n, k;
  int lda, ldb, ldc;
  int tiles_m, tiles_n;
  int k_tiles_per_split;
  int accumulate;      // only honoured when writing the final output
  const float* bias;   // per-column bias added to the final output (or null)
  int vec_out;         // C (and the bias) take 128-bit stores: n, ldc % 4 == 0, 16-byte aligned
  int relu;            // with a bias: ReLU after it (Linear followed by ReLU)
  float* colsum;       // column sums of op(B) (+)= into it (or null): tiny kernel and LDS
                       // tiles with B untransposed and K unsplit
  int colsum_acc;
  const float* bmask;  // tiny kernel, B untransposed: B[k][j] counts only where
                       // 0 < bmask[k][j] < +inf (ReLU's backward mask; same layout as B)
  int walk_a, walk_b;  // short-K kernel: 0, or the XCD-block grid walk_a x walk_b
};

// ReLU's backward mask on a gradient value: ClampBackward's strict bounds for
// clamp(t, 0, DBL_MAX) in float32, t in (0, +inf) keeps g, anything else
// (including NaN) gives +0.0.
__device__ __forceinline__ float relu_masked(float g, float t) {
  return (t > 0.0f && t < __builtin_huge_valf()) ? g : 0.0f;
}

// Linear's epilogue: v + b, then, when asked, ReLU as the clamp functor
// computes clamp(t, 0, +inf) in float32: t < 0 ? 0 : t (NaN and -0.0 pass).
__device__ __forceinline__ float lin_epi(float v, float b, int relu) {
  const float t = v + b;
  return relu && t < 0.0f ? 0.0f : t;
}
__device__ __forceinline__ v4f lin_epi4(v4f v, v4f b, int relu) {
  return v4f{lin_epi(v.x, b.x, relu), lin_epi(v.y, b.y, relu), lin_epi(v.z, b.z, relu),
             lin_epi(v.w, b.w, relu)};
}

// Load one [rows x cols] panel of a row-major matrix (leading dim ld) starting
// at (r0, c0) into registers as float4, bounds-checked against (R, Cn).
// VEC requires ld % 4 == 0, 16-byte base alignment and Cn % 4 == 0, so each
// float4 is either fully inside or fully outside.
template <int ROWS, int COLS, bool VEC>
struct Panel {
  static constexpr int kVec = ROWS * COLS / 4;
  static constexpr int kPer = kVec / kThreads;
  static_assert(kVec % kThreads == 0, "panel must split evenly over threads");
  v4f v[kPer];

  __device__ __forceinline__ void load(const float* __restrict__ p, int ld,
                                       int r0, int c0, int R, int Cn) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int f = threadIdx.x + j * kThreads;
      const int r = f / (COLS / 4);
      const int c = (f % (COLS / 4)) * 4;
      const int gr = r0 + r, gc = c0 + c;
      if constexpr (VEC) {
        if (gr < R && gc < Cn)
          v[j] = *reinterpret_cast<const v4f*>(p + int64_t(gr) * ld + gc);
        else
          v[j] = v4f(0.0f);
      } else {
        const float* q = p + int64_t(gr) * ld + gc;
        v[j].x = (gr < R && gc + 0 < Cn) ? q[0] : 0.0f;
        v[j].y = (gr < R && gc + 1 < Cn) ? q[1] : 0.0f;
        v[j].z = (gr < R && gc + 2 < Cn) ? q[2] : 0.0f;
        v[j].w = (gr < R && gc + 3 < Cn) ? q[3] : 0.0f;
      }
    }
  }
  // Store to an LDS array with row pitch COLS + kPad.
  __device__ __forceinline__ void store(float* lds) const {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int f = threadIdx.x + j * kThreads;
      const int r = f / (COLS / 4);
      const int c = (f % (COLS / 4)) * 4;
      *reinterpret_cast<v4f*>(lds + r * (COLS + kPad) + c) = v[j];
    }
  }
};

template <class C, bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_mfma(GemmArgs g) {
  constexpr int BM = C::BM, BN = C::BN;
  constexpr int HK = kBK / 2;
  constexpr int A_SZ = a_lds_floats<C, TA>();
  constexpr int B_SZ = b_lds_floats<C, TB>();
  __shared__ __attribute__((aligned(16))) float smem[2 * (A_SZ + B_SZ)];

  // XCD-aware regrouping of the tile id, then grouped tile-row walk.
  const int ntiles = g.tiles_m * g.tiles_n;
  int bid = blockIdx.x;
  if (ntiles % 8 == 0) bid = (bid % 8) * (ntiles / 8) + bid / 8;
  constexpr int kGroup = 8;
  const int per_group = kGroup * g.tiles_n;
  const int group = bid / per_group;
  const int first_m = group * kGroup;
  const int gsize = min(g.tiles_m - first_m, kGroup);
  const int in_group = bid - group * per_group;
  const int tile_m = first_m + in_group % gsize;
  const int tile_n = in_group / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int split = blockIdx.z;
  const int k_tiles = (g.k + kBK - 1) / kBK;
  const int kt0 = split * g.k_tiles_per_split;
  const int kt1 = min(k_tiles, kt0 + g.k_tiles_per_split);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int li = lane & 31, lh = lane >> 5;

  // A panel: !TA -> [BM rows of m] x [BK cols of k]; TA -> [BK rows] x [BM cols]
  using PA = std::conditional_t<TA, Panel<kBK, BM, VEC>, Panel<BM, kBK, VEC>>;
  using PB = std::conditional_t<TB, Panel<BN, kBK, VEC>, Panel<kBK, BN, VEC>>;
  PA pa;
  PB pb;

  auto load_tile = [&](int kt) {
    const int k0 = kt * kBK;
    if constexpr (TA) pa.load(g.a, g.lda, k0, m0, g.k, g.m);
    else pa.load(g.a, g.lda, m0, k0, g.m, g.k);
    if constexpr (TB) pb.load(g.b, g.ldb, n0, k0, g.n, g.k);
    else pb.load(g.b, g.ldb, k0, n0, g.k, g.n);
  };

  v16f acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = v16f(0.0f);

  if (kt0 < kt1) {
    load_tile(kt0);
    pa.store(smem);
    pb.store(smem + A_SZ);
  }
  __syncthreads();

  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const float* As = smem + cur * (A_SZ + B_SZ);
    const float* Bs = As + A_SZ;
    const bool more = kt + 1 < kt1;
    if (more) load_tile(kt + 1);

    // Fragments: a[i][s] = A_tile[row_i][s + lh*HK], b[j][s] likewise.
    float af[C::TM][HK], bf[C::TN][HK];
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int row = (wm * C::TM + i) * 32 + li;
      if constexpr (!TA) {
        const float* src = As + row * (kBK + kPad) + lh * HK;
#pragma unroll
        for (int q = 0; q < HK / 4; ++q) {
          const v4f t = *reinterpret_cast<const v4f*>(src + 4 * q);
          af[i][4 * q + 0] = t.x;
          af[i][4 * q + 1] = t.y;
          af[i][4 * q + 2] = t.z;
          af[i][4 * q + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int s = 0; s < HK; ++s) af[i][s] = As[(s + lh * HK) * (BM + kPad) + row];
      }
    }
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int col = (wn * C::TN + j) * 32 + li;
      if constexpr (TB) {
        const float* src = Bs + col * (kBK + kPad) + lh * HK;
#pragma unroll
        for (int q = 0; q < HK / 4; ++q) {
          const v4f t = *reinterpret_cast<const v4f*>(src + 4 * q);
          bf[j][4 * q + 0] = t.x;
          bf[j][4 * q + 1] = t.y;
          bf[j][4 * q + 2] = t.z;
          bf[j][4 * q + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int s = 0; s < HK; ++s) bf[j][s] = Bs[(s + lh * HK) * (BN + kPad) + col];
      }
    }
#pragma unroll
    for (int s = 0; s < HK; ++s)
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s],
                                                           acc[i][j], 0, 0, 0);

    if (more) {
      float* nxt = smem + (cur ^ 1) * (A_SZ + B_SZ);
      pa.store(nxt);
      pb.store(nxt + A_SZ);
    }
    __syncthreads();
  }

  // Epilogue.
  const bool partial = gridDim.z > 1;
  float* out = g.c;
  int64_t ld = g.ldc;
  if (partial) {
    out = g.c + int64_t(split) * g.m * g.n;
    ld = g.n;
  }
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int col = n0 + (wn * C::TN + j) * 32 + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + (wm * C::TM + i) * 32 + (r / 4) * 8 + lh * 4 + (r % 4);
        if (row < g.m && col < g.n) {
          float* p = out + int64_t(row) * ld + col;
          const float v = acc[i][j][r];
          if (!partial && g.accumulate) *p = *p + v;
          else if (!partial && g.bias) *p = lin_epi(v, g.bias[col], g.relu);
          else *p = v;
        }
      }
    }
  }
}

// c[row, col] (+)= sum over splits of part[s, row, col], in split order.
__global__ __launch_bounds__(256) void fold_splits(float* __restrict__ c,
                                                   const float* __restrict__ part,
                                                   int m, int n, int ldc,
                                                   int splits, int accumulate,
                                                   const float* __restrict__ bias, int relu) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t mn = int64_t(m) * n;
  if (i >= mn) return;
  const int row = int(i / n), col = int(i - int64_t(row) * n);
  float acc = part[i];
  for (int s = 1; s < splits; ++s) acc += part[int64_t(s) * mn + i];
  float* p = c + int64_t(row) * ldc + col;
  if (accumulate) *p = *p + acc;
  else *p = bias ? lin_epi(acc, bias[col], relu) : acc;
}

// The same fold, four adjacent columns per lane (n and ldc multiples of four,
// C and the bias 16-byte aligned), the split loads issued four at a time; the
// adds keep split order, so the result equals fold_splits bit for bit.
// col_blocks == 0: lanes take consecutive float4s of C.  col_blocks > 0 (a
// grid of col_blocks x ceil(m / 8) workgroups): workgroup b takes rows
// 8 (b / col_blocks) .. + 7 of the 128 columns of block b % col_blocks, the
// block a split-K workgroup of the same index mod 8 wrote, so the partials
// are read on the XCD whose L2 holds them.
__global__ __launch_bounds__(256) void fold_splits4(float* __restrict__ c,
                                                    const float* __restrict__ part,
                                                    int m, int n, int ldc,
                                                    int splits, int accumulate,
                                                    const float* __restrict__ bias, int relu,
                                                    int col_blocks) {
  int64_t i4;
  if (col_blocks > 0) {
    const int blk = int(blockIdx.x) % col_blocks, sub = int(blockIdx.x) / col_blocks;
    const int r = sub * 8 + int(threadIdx.x >> 5), cl = blk * 128 + 4 * int(threadIdx.x & 31);
    if (r >= m || cl >= n) return;
    i4 = (int64_t(r) * n + cl) / 4;
  } else {
    i4 = int64_t(blockIdx.x) * 256 + threadIdx.x;
  }
  const int64_t mn4 = int64_t(m) * n / 4;
  if (i4 >= mn4) return;
  const int64_t i = 4 * i4;
  const int row = int(i / n), col = int(i - int64_t(row) * n);
  const v4f* src = reinterpret_cast<const v4f*>(part) + i4;
  v4f acc = src[0];
  int s = 1;
  for (; s + 4 <= splits; s += 4) {
    v4f x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = src[int64_t(s + u) * mn4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = acc + x[u];
  }
  for (; s < splits; ++s) acc = acc + src[int64_t(s) * mn4];
  v4f* p = reinterpret_cast<v4f*>(c + int64_t(row) * ldc + col);
  if (accumulate) *p = *p + acc;
  else *p = bias ? lin_epi4(acc, *reinterpret_cast<const v4f*>(bias + col), relu) : acc;
}

// Where split-K partials live: the pool (taken per call and returned once
// the fold is enqueued; stream order makes the reuse safe) or, for the
// no-allocation entry point, the device's fixed workspace.
struct Workspace {
  float* fixed = nullptr;  // device address of the fixed workspace, or null
  size_t fixed_bytes = 0;

  int take(size_t bytes, float** out) const {
    if (fixed) {
      if (bytes > fixed_bytes)
        return fail(LMP_ERR_UNSUPPORTED,
                    "gemm_noalloc: the split-K partials need " + std::to_string(bytes) +
                        " bytes, above the " + std::to_string(fixed_bytes) +
                        "-byte no-allocation workspace (lmp_k_gemm_f32 serves this product)");
      *out = fixed;
      return LMP_OK;
    }
    *out = static_cast<float*>(scratch_alloc(bytes));
    return *out ? LMP_OK : LMP_ERR_OOM;
  }
  void give(float* p) const {
    if (!fixed) scratch_free(p);
  }
};

bool aligned16(const void* p);

// Adds the split-K partials into C (with the epilogue of the final output).
// col_blocks > 0: the partials come in blocks of 128 columns whose splits ran
// on one XCD (see fold_splits4).
int launch_fold(Runtime* rt, float* c, const float* part, int m, int n, int ldc, int splits,
                int accumulate, const float* bias, int relu, int col_blocks = 0) {
  const int64_t mn = int64_t(m) * n;
  if (n % 4 == 0 && ldc % 4 == 0 && aligned16(c) && aligned16(part) &&
      (!bias || aligned16(bias))) {
    const int64_t grid = col_blocks > 0 ? int64_t(col_blocks) * ((m + 7) / 8) : (mn / 4 + 255) / 256;
    hipLaunchKernelGGL(fold_splits4, dim3(uint32_t(grid)), dim3(256), 0, rt->stream, c, part, m,
                       n, ldc, splits, accumulate, bias, relu, col_blocks);
  } else {
    hipLaunchKernelGGL(fold_splits, dim3(uint32_t((mn + 255) / 256)), dim3(256), 0,
                       rt->stream, c, part, m, n, ldc, splits, accumulate, bias, relu);
  }
  LMP_LAUNCH_CHECK("fold_splits");
  return LMP_OK;
}

// ------------------------------------------------------------------ direct
//
// Register-direct MFMA kernel for M <= 32 (a Linear layer at a small batch:
// the weight panel streams once from HBM and nothing is reused enough to pay
// for LDS staging).  Every wave loads its MFMA
// operands straight from global memory in operand layout, 8 values of k per
// iteration.  MFMA step s (0..3) pairs k0 + s (lanes 0-31) with k0 + 4 + s
// (lanes 32-63), so a lane's four A values of one iteration are contiguous in
// k.  A wave owns a 32 x 128 block of C as four 32x32 MFMA blocks q:
//   TB == false: a B row is read as float4 along n, lane c holding columns
//     4c..4c+3; block q takes component q, so block q's column j is
//     n0 + 4j + q and the epilogue writes whole float4s of a row.
//   TB == true: block q covers columns n0 + 32q + (0..31); a lane reads the
//     four k values of one stored B row as one float4.
// The four waves of a workgroup take consecutive quarters of its K range and
// add their blocks in a fixed order through LDS; workgroups split K further
// over blockIdx.y into partials that fold_splits adds in split order.
// Requirements (checked by the host): the contiguous extent of each operand
// is a multiple of four with 16-byte aligned rows, and for TB == false C's
// rows are 16-byte aligned too.
struct DirectArgs {
  const float* a;
  const float* b;
  float* c;  // final output (one split) or partial buffer base
  int m, n, k;
  int lda, ldb, ldc;
  int n_blocks;    // ceil(n / 128)
  int k_per_wg;    // K range of one workgroup (a multiple of 32)
  int accumulate;  // only honoured when writing the final output
  const float* bias;  // per-column bias added to the final output (or null)
  int relu;           // with a bias: ReLU after it
};

constexpr int kDirectN = 128;

// Read by lanes whose operand element lies outside the matrix: zeros, never
// written.
__device__ __attribute__((aligned(16))) float g_direct_zeros[4];

template <bool TA, bool TB>
struct DirectFrag {
  v4f a;     // A values of steps 0..3
  v4f b[4];  // TB: b[q][s]; !TB: b[s][q]

  // Loads are unconditional: a lane whose element lies outside the matrix (or
  // past ke) reads zeros from g_direct_zeros instead.  B (the weight, read
  // once) is loaded with the nontemporal hint so it does not push A out of
  // the L2.  Guarded loads would
  // each sit behind a branch, and a select after the load would wait for it
  // at once; either way nothing would stay in flight while the MFMAs run.
  __device__ __forceinline__ void load(const DirectArgs& g, int row, int n0, int k0,
                                       int ke, int li, int lh) {
    const int kq = k0 + 4 * lh;  // first k of this lane's half
    if constexpr (!TA) {
      const bool ok = row < g.m && kq < ke;
      a = *reinterpret_cast<const v4f*>(ok ? g.a + int64_t(row) * g.lda + kq
                                           : g_direct_zeros);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bool ok = row < g.m && kq + s < ke;
        a[s] = *(ok ? g.a + int64_t(kq + s) * g.lda + row : g_direct_zeros);
      }
    }
    if constexpr (!TB) {
      const int col = n0 + 4 * li;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bool ok = col < g.n && kq + s < ke;
        b[s] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(
            ok ? g.b + int64_t(kq + s) * g.ldb + col : g_direct_zeros));
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = n0 + 32 * q + li;
        const bool ok = col < g.n && kq < ke;
        b[q] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(
            ok ? g.b + int64_t(col) * g.ldb + kq : g_direct_zeros));
      }
    }
  }

  __device__ __forceinline__ void mma(v16f (&acc)[4]) const {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc[q] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], TB ? b[q][s] : b[s][q],
                                                      acc[q], 0, 0, 0);
  }
};

// Output row of accumulator register r for a lane in half lh (0 or 1).
__device__ __forceinline__ int direct_row(int r, int lh) {
  return (r / 4) * 8 + lh * 4 + (r % 4);
}

constexpr int kDirectWaves = 4;

template <bool TA, bool TB, int STAGES>
__global__ __launch_bounds__(64 * kDirectWaves)
__attribute__((amdgpu_waves_per_eu(STAGES > 2 ? 2 : TB ? 3 : 4)))
void gemm_direct(DirectArgs g) {
  constexpr int KW = kDirectWaves;
  // The wave index (and with it the K range) is uniform across the wave;
  // saying so keeps the K loop a scalar loop.
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int li = lane & 31, lh = lane >> 5;
  const int n0 = int(blockIdx.x % g.n_blocks) * kDirectN;
  const int part = g.k_per_wg / KW;
  const int kb = int(blockIdx.y) * g.k_per_wg + wave * part;
  const int ke = min(g.k, kb + part);

  v16f acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) acc[q] = v16f(0.0f);

  // STAGES fragments in flight: each iteration's loads are issued STAGES - 1
  // iterations ahead of its MFMAs.  Loads at or past ke yield zeros, so the
  // tail needs no branch (0 * 0 adds nothing).
  DirectFrag<TA, TB> f[STAGES];
#pragma unroll
  for (int s = 0; s < STAGES; ++s) f[s].load(g, li, n0, kb + 8 * s, ke, li, lh);
  for (int k0 = kb; k0 < ke; k0 += 8 * STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
      f[s].mma(acc);
      // Keep each refill right after the MFMAs that free its registers; the
      // scheduler would otherwise sink every load to the end of the trip,
      // leaving nothing in flight while the MFMAs run.
      __builtin_amdgcn_sched_barrier(0);
      f[s].load(g, li, n0, k0 + 8 * (s + STAGES), ke, li, lh);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  const bool partial = gridDim.y > 1;
  float* out = partial ? g.c + int64_t(blockIdx.y) * g.m * g.n : g.c;
  const int64_t ld = partial ? int64_t(g.n) : int64_t(g.ldc);
  const bool acc_out = !partial && g.accumulate;
  const float* bias = partial ? nullptr : g.bias;

  // Blocks are added over the waves through LDS in rounds of BPR blocks
  // (32 KiB), laid out [wave][block][r][lane] so writes and reads are
  // conflict-free.  Thread t owns the (r, lane) pairs p = t + 64*KW*u and
  // sums them in wave order.
  constexpr int BPR = 8 / KW, U = 16 / KW, NT = 64 * KW;
  __shared__ __attribute__((aligned(16))) float red[KW * BPR * 16 * 64];
  v4f v[U];
#pragma unroll
  for (int round = 0; round < 4 / BPR; ++round) {
    if (round) __syncthreads();
#pragma unroll
    for (int qq = 0; qq < BPR; ++qq)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        red[((wave * BPR + qq) * 16 + r) * 64 + lane] = acc[round * BPR + qq][r];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = int(threadIdx.x) + NT * u;
      const int r = p >> 6, ln = p & 63;
#pragma unroll
      for (int qq = 0; qq < BPR; ++qq) {
        float t = red[(qq * 16 + r) * 64 + ln];
#pragma unroll
        for (int w = 1; w < KW; ++w) t += red[((w * BPR + qq) * 16 + r) * 64 + ln];
        v[u][round * BPR + qq] = t;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int p = int(threadIdx.x) + NT * u;
    const int r = p >> 6, ln = p & 63;
    const int orow = direct_row(r, ln >> 5);
    if (orow >= g.m) continue;
    float* base = out + int64_t(orow) * ld;
    if constexpr (!TB) {
      const int col = n0 + 4 * (ln & 31);
      if (col < g.n) {
        v4f* o = reinterpret_cast<v4f*>(base + col);
        if (acc_out) *o = *o + v[u];
        else if (bias) *o = lin_epi4(v[u], *reinterpret_cast<const v4f*>(bias + col), g.relu);
        else *o = v[u];
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = n0 + 32 * q + (ln & 31);
        if (col < g.n) {
          if (acc_out) base[col] = base[col] + v[u][q];
          else base[col] = bias ? lin_epi(v[u][q], bias[col], g.relu) : v[u][q];
        }
      }
    }
  }
}

// ------------------------------------------------------------------ tiny
//
// Latency-bound GEMMs (up to about two million multiply-adds with K <= 512,
// e.g. the README MLP's layers): one workgroup per BS x BS block of C (BS =
// 32 with 32x32x2 MFMAs, or 16 with 16x16x4 MFMAs when 32-wide blocks would
// leave most CUs idle), its four waves taking consecutive quarters of K in
// groups of G = 4 * (64 / BS) k values and adding their blocks through LDS
// in wave order.  Lane l holds row / column l % BS; within group j, MFMA step
// s (0..3) gives lane part q = l / BS the k value G*j + 4q + s, so a lane's
// four values of an operand whose k is contiguous in memory (A untransposed,
// B transposed) are one 128-bit load when the rows allow it; the other
// operand is read a k value per load, consecutive lanes reading consecutive
// addresses.  All of a wave's loads are issued before its first MFMA, so a
// block costs about one memory latency plus the wave's MFMAs, where the tiled
// kernels pay a pipeline fill per K tile and the register-direct kernel a
// 32x128 block per wave.
//
// Operands are read through buffer resources: an offset at or past the
// resource's size (kTinyOob) reads zero, so rows or columns outside the matrix
// and k past the wave's range cost one select each.
constexpr int64_t kTinyMaxMacs = int64_t(1) << 21;
constexpr int kTinyMaxK = 512;
constexpr uint32_t kTinyOob = 0x80000000u;
constexpr uint32_t kTinyMaxBytes = 1u << 30;  // operand extents stay below kTinyOob

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tiny_rsrc(const float* p, uint32_t bytes) {
  // Third dword 0x00020000: a raw 32-bit buffer on gfx9-family targets.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, int(bytes), 0x00020000);
}

// One operand of one lane: `base` is the byte offset of the lane's row of
// op(A) or column of op(B) (kTinyOob outside the matrix), `kstep` the byte
// distance between consecutive k.  VEC: k is contiguous and rows are 16-byte
// multiples, K % 4 == 0, so a lane's four k values of a group come in one
// load that is either wholly inside or wholly past K.
template <bool VEC>
struct TinyOperand {
  __amdgpu_buffer_rsrc_t r;
  uint32_t base, kstep;
  __device__ __forceinline__ v4f load(int k, int kend) const {  // k, k+1, k+2, k+3
    v4f v;
    if constexpr (VEC) {
      const uint32_t o = k < kend ? base + 4u * uint32_t(k) : kTinyOob;
      v = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, int(o), 0, 0));
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t o = k + s < kend ? base + uint32_t(k + s) * kstep : kTinyOob;
        v[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, int(o), 0, 0));
      }
    }
    return v;
  }
};

template <int BS>
struct TinyMma;
template <>
struct TinyMma<32> {
  using Acc = v16f;
  static constexpr int kRegs = 16;
  __device__ __forceinline__ static Acc step(float a, float b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  // Row of accumulator register r for lane part q (l / 32).
  __device__ __forceinline__ static int row(int r, int q) { return direct_row(r, q); }
};
template <>
struct TinyMma<16> {
  using Acc = v4f;
  static constexpr int kRegs = 4;
  __device__ __forceinline__ static Acc step(float a, float b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static int row(int r, int q) { return q * 4 + r; }
};

// One BS x BS block (bx, by) of C = op(A) op(B) by the tiny kernel's four
// waves; red holds 4 * TinyMma<BS>::kRegs * 64 floats, red_cs 4 * 64.
template <int BS, bool TA, bool TB, bool VA, bool VB, bool MB>
__device__ __forceinline__ void tiny_block(const GemmArgs& g, int bx, int by, float* red,
                                           float* red_cs) {
  static_assert(!MB || !TB, "the B mask is for B untransposed");
  using M = TinyMma<BS>;
  constexpr int G = 4 * (64 / BS);              // k values per group
  constexpr int kGroups = kTinyMaxK / G / 4;    // a wave's quarter of K <= 512
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int li = lane % BS, q = lane / BS;
  const int m0 = bx * BS, n0 = by * BS;
  const int groups = (g.k + G - 1) / G;
  const int per = (groups + 3) / 4;
  const int j0 = min(groups, wave * per), j1 = min(groups, j0 + per);
  const int kend = min(g.k, G * j1);
  // Stored extents: A is [k, m] (TA) or [m, k]; B is [n, k] (TB) or [k, n].
  const uint32_t a_bytes = 4u * uint32_t(TA ? (g.k - 1) * g.lda + g.m : (g.m - 1) * g.lda + g.k);
  const uint32_t b_bytes = 4u * uint32_t(TB ? (g.n - 1) * g.ldb + g.k : (g.k - 1) * g.ldb + g.n);
  const int row = m0 + li, col = n0 + li;
  const TinyOperand<VA> opa{tiny_rsrc(g.a, a_bytes),
                            row < g.m ? 4u * uint32_t(TA ? row : row * g.lda) : kTinyOob,
                            TA ? 4u * uint32_t(g.lda) : 4u};
  const uint32_t b_base = col < g.n ? 4u * uint32_t(TB ? col * g.ldb : col) : kTinyOob;
  const uint32_t b_kstep = TB ? 4u : 4u * uint32_t(g.ldb);
  const TinyOperand<VB> opb{tiny_rsrc(g.b, b_bytes), b_base, b_kstep};
  // Every load of the wave's range is issued before the first MFMA (group
  // branches are uniform), so the range costs one memory latency.
  v4f a[kGroups], b[kGroups];
#pragma unroll
  for (int c = 0; c < kGroups; ++c)
    if (j0 + c < j1) {
      a[c] = opa.load(G * (j0 + c) + 4 * q, kend);
      b[c] = opb.load(G * (j0 + c) + 4 * q, kend);
    }
  if constexpr (MB) {
    // The mask has B's layout: the same offsets, loaded beside B; values
    // past the matrix read 0 and mask to 0, as B's do.
    const TinyOperand<VB> opm{tiny_rsrc(g.bmask, b_bytes), b_base, b_kstep};
    v4f mk[kGroups];
#pragma unroll
    for (int c = 0; c < kGroups; ++c)
      if (j0 + c < j1) mk[c] = opm.load(G * (j0 + c) + 4 * q, kend);
#pragma unroll
    for (int c = 0; c < kGroups; ++c)
      if (j0 + c < j1)
#pragma unroll
        for (int s = 0; s < 4; ++s) b[c][s] = relu_masked(b[c][s], mk[c][s]);
  }
  typename M::Acc acc = typename M::Acc(0.0f);
#pragma unroll
  for (int c = 0; c < kGroups; ++c)
    if (j0 + c < j1)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = M::step(a[c][s], b[c][s], acc);
  // Column sums of op(B) (a Linear's bias gradient beside its weight
  // gradient): the first row of blocks adds the B values its lanes already
  // hold -- each lane its k values in order, then the lane parts and the
  // waves in order through LDS.  Sums start from +0, so -0.0 never appears.
  const bool colsum = g.colsum != nullptr && bx == 0;
  if (colsum) {
    float cs = 0.0f;
#pragma unroll
    for (int c = 0; c < kGroups; ++c)
      if (j0 + c < j1)
#pragma unroll
        for (int s = 0; s < 4; ++s) cs += b[c][s];
    red_cs[wave * 64 + lane] = cs;  // [wave][part q][column li]
  }
  // Blocks of the four waves summed in wave order: [wave][r][lane].
  constexpr int R = M::kRegs;
#pragma unroll
  for (int r = 0; r < R; ++r) red[(wave * R + r) * 64 + lane] = acc[r];
  __syncthreads();
  if (colsum && int(threadIdx.x) < BS) {
    const int col = n0 + int(threadIdx.x);
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
      for (int qq = 0; qq < 64 / BS; ++qq) v += red_cs[w * 64 + qq * BS + int(threadIdx.x)];
    if (col < g.n) g.colsum[col] = g.colsum_acc ? g.colsum[col] + v : v;
  }
#pragma unroll
  for (int u = 0; u < R / 4; ++u) {
    const int p = int(threadIdx.x) + 256 * u;  // (r, lane) pair
    const int r = p >> 6, ln = p & 63;
    float v = red[p];
#pragma unroll
    for (int w = 1; w < 4; ++w) v += red[w * R * 64 + p];
    const int orow = m0 + M::row(r, ln / BS), ocol = n0 + ln % BS;
    if (orow >= g.m || ocol >= g.n) continue;
    float* o = g.c + int64_t(orow) * g.ldc + ocol;
    if (g.accumulate) *o = *o + v;
    else *o = g.bias ? lin_epi(v, g.bias[ocol], g.relu) : v;
  }
}

template <int BS, bool TA, bool TB, bool VA, bool VB, bool MB = false>
__global__ __launch_bounds__(256) void gemm_tiny(GemmArgs g) {
  __shared__ float red[4 * TinyMma<BS>::kRegs * 64];
  __shared__ float red_cs[4 * 64];
  tiny_block<BS, TA, TB, VA, VB, MB>(g, int(blockIdx.x), int(blockIdx.y), red, red_cs);
}

// A Linear's three gradients in one launch, on 16 x 16 blocks: workgroups
// below wblocks take a block of dW = X^T G (A = X stored [batch, in]) with the
// column sums of G as db; the rest a block of dX = G W^T (B = W stored
// [in, out]).  Each block is the tiny kernel's, so every output has the bits
// of the two separate launches.
template <bool VA, bool VB>
__global__ __launch_bounds__(256) void gemm_tiny_linear_backward(GemmArgs gw, GemmArgs gx,
                                                                 int wblocks_m, int wblocks) {
  __shared__ float red[4 * TinyMma<16>::kRegs * 64];
  __shared__ float red_cs[4 * 64];
  const int b = int(blockIdx.x);
  if (b < wblocks) {
    tiny_block<16, true, false, false, false, false>(gw, b % wblocks_m, b / wblocks_m, red,
                                                      red_cs);
  } else {
    const int t = b - wblocks, xm = (gx.m + 15) / 16;
    tiny_block<16, false, true, VA, VB, false>(gx, t % xm, t / xm, red, red_cs);
  }
}

bool tiny_ok(const GemmArgs& g) {
  if (g.k > kTinyMaxK || int64_t(g.m) * g.n * g.k > kTinyMaxMacs) return false;
  const int64_t a_elems = int64_t(g.lda) * (g.k > g.m ? g.k : g.m);  // bounds either layout
  const int64_t b_elems = int64_t(g.ldb) * (g.k > g.n ? g.k : g.n);
  return 4 * a_elems < kTinyMaxBytes && 4 * b_elems < kTinyMaxBytes;
}

bool aligned16(const void* p);

template <int BS, bool TA, bool TB>
void launch_tiny_bs(Runtime* rt, const GemmArgs& g, bool va, bool vb) {
  const dim3 grid{uint32_t((g.m + BS - 1) / BS), uint32_t((g.n + BS - 1) / BS), 1u};
  if constexpr (!TB) {
    if (g.bmask) {  // B is never 128-bit along k here (k strides by ldb)
      if (va)
        hipLaunchKernelGGL((gemm_tiny<BS, TA, TB, !TA, false, true>), grid, dim3(256), 0,
                           rt->stream, g);
      else
        hipLaunchKernelGGL((gemm_tiny<BS, TA, TB, false, false, true>), grid, dim3(256), 0,
                           rt->stream, g);
      return;
    }
  }
  if (va && vb)
    hipLaunchKernelGGL((gemm_tiny<BS, TA, TB, !TA, TB>), grid, dim3(256), 0, rt->stream, g);
  else if (va)
    hipLaunchKernelGGL((gemm_tiny<BS, TA, TB, !TA, false>), grid, dim3(256), 0, rt->stream, g);
  else if (vb)
    hipLaunchKernelGGL((gemm_tiny<BS, TA, TB, false, TB>), grid, dim3(256), 0, rt->stream, g);
  else
    hipLaunchKernelGGL((gemm_tiny<BS, TA, TB, false, false>), grid, dim3(256), 0, rt->stream,
                       g);
}

template <bool TA, bool TB>
int launch_tiny(Runtime* rt, const GemmArgs& g) {
  // 128-bit k loads for an operand whose k is contiguous, with 16-byte rows.
  const bool k4 = g.k % 4 == 0;
  const bool va = !TA && k4 && g.lda % 4 == 0 && aligned16(g.a);
  const bool vb = TB && k4 && g.ldb % 4 == 0 && aligned16(g.b);
  // 16x16 blocks unless 32x32 blocks already cover a quarter of the CUs.
  const int64_t blocks32 = int64_t((g.m + 31) / 32) * ((g.n + 31) / 32);
  if (blocks32 * 4 >= rt->cu_count) launch_tiny_bs<32, TA, TB>(rt, g, va, vb);
  else launch_tiny_bs<16, TA, TB>(rt, g, va, vb);
  LMP_LAUNCH_CHECK("gemm_tiny");
  return LMP_OK;
}

// Whether launch_tiny would run g on 16 x 16 blocks.
bool tiny16(const Runtime* rt, const GemmArgs& g) {
  const int64_t blocks32 = int64_t((g.m + 31) / 32) * ((g.n + 31) / 32);
  return tiny_ok(g) && blocks32 * 4 < rt->cu_count;
}

// gw: dW = X^T G with db (launch_tiny<true, false>); gx: dX = G W^T
// (launch_tiny<false, true>), both on 16 x 16 blocks, in one grid.
int launch_tiny_linear_backward(Runtime* rt, const GemmArgs& gw, const GemmArgs& gx) {
  const bool k4 = gx.k % 4 == 0;
  const bool va = k4 && gx.lda % 4 == 0 && aligned16(gx.a);
  const bool vb = k4 && gx.ldb % 4 == 0 && aligned16(gx.b);
  const int wm = (gw.m + 15) / 16, wblocks = wm * ((gw.n + 15) / 16);
  const int xblocks = ((gx.m + 15) / 16) * ((gx.n + 15) / 16);
  const dim3 grid{uint32_t(wblocks + xblocks)};
  if (va && vb)
    hipLaunchKernelGGL((gemm_tiny_linear_backward<true, true>), grid, dim3(256), 0, rt->stream,
                       gw, gx, wm, wblocks);
  else if (va)
    hipLaunchKernelGGL((gemm_tiny_linear_backward<true, false>), grid, dim3(256), 0, rt->stream,
                       gw, gx, wm, wblocks);
  else if (vb)
    hipLaunchKernelGGL((gemm_tiny_linear_backward<false, true>), grid, dim3(256), 0, rt->stream,
                       gw, gx, wm, wblocks);
  else
    hipLaunchKernelGGL((gemm_tiny_linear_backward<false, false>), grid, dim3(256), 0,
                       rt->stream, gw, gx, wm, wblocks);
  LMP_LAUNCH_CHECK("gemm_tiny_linear_backward");
  return LMP_OK;
}

// ------------------------------------------------------------- LDS-direct
//
// Tile kernels for operands that allow 128-bit loads.  Panels go from global
// memory straight into LDS with global_load_lds_dwordx4 (no VGPR staging and
// no ds_write) through a STAGES-deep ring with one barrier per K tile: at the
// top of tile t every wave waits for its own loads of tile t, the barrier
// makes all of them visible (and retires every wave's reads of the stage about
// to be refilled), then the loads of tile t + STAGES - 1 are issued.  Within a
// tile the four 4-step sub-steps are software-pipelined: the LDS fragments of
// sub-step u+1 are read while the MFMAs of sub-step u run.  Each wave owns
// TM x TN blocks of 32x32 in a WM x WN grid of waves.  Tile walk, MFMA step
// order and epilogue are those of gemm_f32_mfma, so every configuration
// produces the same bits for the same split of K.
//
// One DMA instruction fills a contiguous 1 KiB of LDS (lane i -> bytes 16i..),
// so the LDS layout is chosen by which global float4 each lane fetches:
//   K-major panel (32 k values contiguous in global: A untransposed, B
//     transposed), R rows x 8 chunks of 4 floats: 16-byte slot p holds row
//     p / 8, chunk (p % 8) ^ kswz(row).  A lane's fragment read (one row, one
//     chunk) then spreads 16 consecutive rows over all 64 banks.
//   N-major panel (R m or n values contiguous: A transposed, B untransposed),
//     32 k-rows x R/4 chunks: slot p holds k-row p / (R/4), chunk
//     (p % (R/4)) ^ 8 * (k-row / 16).  Lanes 32-63 read k-rows 16 apart from
//     lanes 0-31; the swizzle moves them to the other half of the banks.
// Lanes whose element lies outside the matrix fetch the zero page.
//
// Configurations (measured on MI355X against the register-staged kernel):
//   LdsSmall  128 x 128, 4 waves, 2 stages, two workgroups per CU
//   LdsWide   256 x 128, 8 waves, 3 stages (144 KiB), for M >= 512 when
//             256 x 256 tiles cannot fill the CUs (K split)
//   LdsBig    256 x 256, 8 waves of 128 x 64, 2 stages (128 KiB), whenever its
//             tiles cover the CUs: 4096^3 130 -> 139 TFLOP/s
//   LdsMid    128 x 64, 4 waves of 32 x 64, 3 stages (72 KiB), K split so the
//             tiles cover the CUs, when 128 x 128 tiles would not (K >= 512):
//             config 4's last layer 512x1000x4096 49.6 -> 45.6 us and
//             512x4096x1000 (B transposed) 46.2 -> 42.3 us, 1024^3 30.7 ->
//             26.3 us (medians of interleaved rounds, random operands)
template <int WM_, int WN_, int TM_, int TN_, int STAGES_, int MINB_>
struct LdsCfg {
  static constexpr int WM = WM_, WN = WN_, TM = TM_, TN = TN_;
  static constexpr int STAGES = STAGES_, MINB = MINB_;
  static constexpr int NW = WM * WN, THREADS = 64 * NW;
  static constexpr int BM = WM * TM * 32, BN = WN * TN * 32;
  static constexpr int A_PANEL = BM * kBK, B_PANEL = BN * kBK;
  static constexpr int STAGE = A_PANEL + B_PANEL;  // floats
  static constexpr int A_DMA = BM * 8 / 64 / NW;   // DMA instructions per wave and tile
  static constexpr int B_DMA = BN * 8 / 64 / NW;
  static_assert(A_DMA * 64 * NW == BM * 8 && B_DMA * 64 * NW == BN * 8, "panels split evenly");
  static_assert(BM >= 64 && BN >= 64, "N-major swizzle needs 16 or more chunks per k-row");
};
using LdsSmall = LdsCfg<2, 2, 2, 2, 2, 2>;
using LdsWide = LdsCfg<4, 2, 2, 2, 3, 1>;
using LdsBig = LdsCfg<2, 4, 4, 2, 2, 1>;
using LdsMid = LdsCfg<4, 1, 1, 2, 3, 1>;


__device__ __forceinline__ int kswz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// One 16-byte global load per lane into LDS.  Kept out of the templates: a
// target builtin inside a kernel template keeps the host pass from emitting
// that kernel's launch stub.
__device__ __forceinline__ void lds_dma16(const float* src, float* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}
// The same with the nontemporal hint (cache-policy bit 1, `nt`): for operand
// lines read once, so they do not push reused lines out of the L2.
__device__ __forceinline__ void lds_dma16_nt(const float* src, float* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 2);
}

// Wait until at most N of this wave's vector-memory operations are
// outstanding (gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14, expcnt
// and lgkmcnt left at their maxima).  The empty asm statements with a memory
// clobber keep the compiler from moving LDS accesses across the wait: the
// LDS a DMA load fills is not visible to its alias analysis.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}

// One workgroup's tile of C (or of its split-K partial): `bid` is the tile's
// index in launch order, `split` the K split, `partial` whether K is split
// (the tile then goes to the partial buffer without epilogue).  `smem` holds
// at least C::STAGES * C::STAGE floats, 1 KiB aligned.
template <class C, bool TA, bool TB>
__device__ __forceinline__ void gemm_f32_lds_tile(const GemmArgs& g, int bid, const int split,
                                                  const bool partial, float* smem) {
  constexpr int NT = C::THREADS;
  constexpr int BM = C::BM, BN = C::BN, TM = C::TM, TN = C::TN, S = C::STAGES;
  constexpr int HK = kBK / 2;
  constexpr int SU = 4;           // MFMA steps per sub-step
  constexpr int NU = HK / SU;     // sub-steps per K tile
  constexpr int DPT = C::A_DMA + C::B_DMA;

  const int ntiles = g.tiles_m * g.tiles_n;
  if (ntiles % 8 == 0) bid = (bid % 8) * (ntiles / 8) + bid / 8;
  constexpr int kGroup = 8;
  const int per_group = kGroup * g.tiles_n;
  const int group = bid / per_group;
  const int first_m = group * kGroup;
  const int gsize = min(g.tiles_m - first_m, kGroup);
  const int in_group = bid - group * per_group;
  const int tile_m = first_m + in_group % gsize;
  const int tile_n = in_group / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int k_tiles = (g.k + kBK - 1) / kBK;
  const int kt0 = split * g.k_tiles_per_split;
  const int kt1 = min(k_tiles, kt0 + g.k_tiles_per_split);

  // Column sums of op(B) beside the product (a Linear's bias gradient beside
  // its weight gradient; the host passes colsum only with B untransposed and
  // K unsplit): the workgroups of the first tile row add up the B panels they
  // stage anyway.  Thread t owns column t % BN of the tile and rows
  // (t / BN) * CS_ROWS .. + CS_ROWS - 1 of every K tile, in K order; the parts
  // are added in part order at the end.
  constexpr int CS_PARTS = NT / BN, CS_ROWS = kBK / CS_PARTS;
  static_assert(TB || (NT % BN == 0 && kBK % CS_PARTS == 0), "column-sum layout");
  const bool do_cs = !TB && g.colsum != nullptr && tile_m == 0;  // uniform per workgroup
  const int cs_col = int(threadIdx.x) % BN, cs_part = int(threadIdx.x) / BN;
  float cs = 0.0f;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int li = lane & 31, lh = lane >> 5;

  // The zero page's address, materialised once outside the loop.
  uint64_t zero_bits = reinterpret_cast<uint64_t>(g_direct_zeros);
  asm volatile("" : "+s"(zero_bits));
  const float* zero = reinterpret_cast<const float*>(zero_bits);

  // Per DMA instruction: the lane's fixed coordinate along m (or n), its k
  // offset inside the tile, and its element offset without the tile's k0.
  int a_mn[C::A_DMA], a_k[C::A_DMA], b_mn[C::B_DMA], b_k[C::B_DMA];
  int64_t a_off[C::A_DMA], b_off[C::B_DMA];
#pragma unroll
  for (int q = 0; q < C::A_DMA; ++q) {
    const int p = (wave * C::A_DMA + q) * 64 + lane;
    if constexpr (!TA) {
      const int r = p >> 3, c = (p & 7) ^ kswz(p >> 3);
      a_mn[q] = m0 + r;
      a_k[q] = 4 * c;
      a_off[q] = int64_t(m0 + r) * g.lda + 4 * c;
    } else {
      constexpr int CH = BM / 4;
      const int kr = p / CH, c = (p % CH) ^ ((kr >> 4) << 3);
      a_mn[q] = m0 + 4 * c;
      a_k[q] = kr;
      a_off[q] = int64_t(kr) * g.lda + m0 + 4 * c;
    }
  }
#pragma unroll
  for (int q = 0; q < C::B_DMA; ++q) {
    const int p = (wave * C::B_DMA + q) * 64 + lane;
    if constexpr (TB) {
      const int r = p >> 3, c = (p & 7) ^ kswz(p >> 3);
      b_mn[q] = n0 + r;
      b_k[q] = 4 * c;
      b_off[q] = int64_t(n0 + r) * g.ldb + 4 * c;
    } else {
      constexpr int CH = BN / 4;
      const int kr = p / CH, c = (p % CH) ^ ((kr >> 4) << 3);
      b_mn[q] = n0 + 4 * c;
      b_k[q] = kr;
      b_off[q] = int64_t(kr) * g.ldb + n0 + 4 * c;
    }
  }
  auto issue = [&](int kt, int stage) {
    const int k0 = kt * kBK;
    float* sa = smem + stage * C::STAGE;
    float* sb = sa + C::A_PANEL;
#pragma unroll
    for (int q = 0; q < C::A_DMA; ++q) {
      const bool ok = a_mn[q] < g.m && k0 + a_k[q] < g.k;
      const float* src = ok ? g.a + a_off[q] + (TA ? int64_t(k0) * g.lda : k0) : zero;
      lds_dma16(src, sa + (wave * C::A_DMA + q) * 256);
    }
#pragma unroll
    for (int q = 0; q < C::B_DMA; ++q) {
      const bool ok = b_mn[q] < g.n && k0 + b_k[q] < g.k;
      const float* src = ok ? g.b + b_off[q] + (TB ? k0 : int64_t(k0) * g.ldb) : zero;
      lds_dma16(src, sb + (wave * C::B_DMA + q) * 256);
    }
  };
  // MFMA operands of sub-step u (steps SU*u .. SU*u+3 of the tile): step s
  // reads k = s + HK*lh, as in gemm_f32_mfma.
  auto read_frag = [&](int stage, int u, float (&fa)[TM][SU], float (&fb)[TN][SU]) {
    const float* sa = smem + stage * C::STAGE;
    const float* sb = sa + C::A_PANEL;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = (wm * TM + i) * 32 + li;
      if constexpr (!TA) {
        const int slot = row * 8 + ((lh * 4 + u) ^ kswz(row));
        const v4f t = *reinterpret_cast<const v4f*>(sa + slot * 4);
        fa[i][0] = t.x; fa[i][1] = t.y; fa[i][2] = t.z; fa[i][3] = t.w;
      } else {
#pragma unroll
        for (int s = 0; s < SU; ++s)
          fa[i][s] = sa[(lh * HK + SU * u + s) * BM + (row ^ (lh << 5))];
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = (wn * TN + j) * 32 + li;
      if constexpr (TB) {
        const int slot = col * 8 + ((lh * 4 + u) ^ kswz(col));
        const v4f t = *reinterpret_cast<const v4f*>(sb + slot * 4);
        fb[j][0] = t.x; fb[j][1] = t.y; fb[j][2] = t.z; fb[j][3] = t.w;
      } else {
#pragma unroll
        for (int s = 0; s < SU; ++s)
          fb[j][s] = sb[(lh * HK + SU * u + s) * BN + (col ^ (lh << 5))];
      }
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16f(0.0f);
  auto mma = [&](const float (&fa)[TM][SU], const float (&fb)[TN][SU]) {
#pragma unroll
    for (int s = 0; s < SU; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
  };

  // Sub-steps alternate between two fragment buffers; the last one of a tile
  // (odd, NU being even) uses fa1/fb1.  Its MFMAs are held back until after
  // the next tile's barrier: they need only registers, so they keep the
  // matrix cores busy while the waves issue that tile's DMA and wait for its
  // first fragments, where the 8 waves of one workgroup would otherwise all
  // stall together.  The MFMA order of every accumulator is unchanged.
  static_assert(NU % 2 == 0, "the last sub-step's fragments are fa1/fb1");
  float fa0[TM][SU], fb0[TN][SU], fa1[TM][SU], fb1[TN][SU];
#pragma unroll
  for (int t = 0; t < S - 1; ++t)
    if (kt0 + t < kt1) issue(kt0 + t, t);
  bool owed = false;  // the previous tile's last sub-step is still to run
  for (int kt = kt0; kt < kt1; ++kt) {
    const int rel = kt - kt0;
    const int stage = rel % S;
    // Tile kt has landed once at most the later tiles' loads are in flight.
    if (kt + S - 2 < kt1) wait_vmcnt<(S - 2) * DPT>();
    else wait_vmcnt<0>();
    // The memory clobber keeps the compiler from moving LDS accesses across.
    asm volatile("s_barrier" ::: "memory");
    // The stage refilled here was last read in the previous iteration, whose
    // reads every wave retired before this barrier (the held-back MFMAs read
    // registers only).
    read_frag(stage, 0, fa0, fb0);
    if (owed) mma(fa1, fb1);
    if (kt + S - 1 < kt1) issue(kt + S - 1, (rel + S - 1) % S);
    // Order for the scheduler (masks: 0x8 MFMA, 0x20 global load, 0x100 LDS
    // read, 0x2 / 0x4 VALU / SALU): the first fragments' LDS reads, then one
    // held-back MFMA per DMA instruction with its address work.
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x006, 6, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u + 1 < NU; ++u) {
      if (u % 2 == 0) {
        read_frag(stage, u + 1, fa1, fb1);
        mma(fa0, fb0);
      } else {
        read_frag(stage, u + 1, fa0, fb0);
        mma(fa1, fb1);
      }
      // The next sub-step's LDS reads one per MFMA among the first of this
      // sub-step's MFMAs, with their address work.
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    owed = true;
    if constexpr (!TB) {
      if (do_cs) {
        const float* sb = smem + stage * C::STAGE + C::A_PANEL;
#pragma unroll
        for (int r = 0; r < CS_ROWS; ++r) {
          const int kr = cs_part * CS_ROWS + r;
          cs += sb[kr * BN + (cs_col ^ ((kr >> 4) << 5))];
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  if (owed) mma(fa1, fb1);

  if constexpr (!TB) {
    if (do_cs) {
      // The parts of each column in part order, once every wave is done with
      // the stages.
      asm volatile("s_barrier" ::: "memory");
      smem[threadIdx.x] = cs;
      __syncthreads();
      if (int(threadIdx.x) < BN) {
        float t = smem[threadIdx.x];
#pragma unroll
        for (int q = 1; q < CS_PARTS; ++q) t += smem[q * BN + threadIdx.x];
        const int col = n0 + int(threadIdx.x);
        if (col < g.n) g.colsum[col] = g.colsum_acc ? g.colsum[col] + t : t;
      }
      __syncthreads();
    }
  }

  float* out = g.c;
  int64_t ld = g.ldc;
  if (partial) {
    out = g.c + int64_t(split) * g.m * g.n;
    ld = g.n;
  }
  const float* bias = partial ? nullptr : g.bias;
  const bool acc_out = !partial && g.accumulate;
  if (g.vec_out) {
    // Rows of C as 128-bit stores: each 32x32 block goes through a wave-private
    // 32 x 36 LDS tile (rows padded to keep float4 alignment) so a lane holds
    // four consecutive columns of one row.  LDS requests of one wave complete
    // in order, so the wave's own writes are visible to its reads.
    asm volatile("s_barrier" ::: "memory");  // every wave is done with the stages
    float* tile = smem + wave * (32 * 36);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          tile[((r / 4) * 8 + lh * 4 + (r % 4)) * 36 + li] = acc[i][j][r];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int row0 = m0 + (wm * TM + i) * 32, col0 = n0 + (wn * TN + j) * 32;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int idx = lane + 64 * t;
          const int rr = idx >> 3, cc = (idx & 7) * 4;
          const v4f v = *reinterpret_cast<const v4f*>(tile + rr * 36 + cc);
          const int row = row0 + rr, col = col0 + cc;
          if (row < g.m && col < g.n) {
            v4f* p = reinterpret_cast<v4f*>(out + int64_t(row) * ld + col);
            if (acc_out) *p = *p + v;
            else if (bias) *p = lin_epi4(v, *reinterpret_cast<const v4f*>(bias + col), g.relu);
            else *p = v;
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + (wn * TN + j) * 32 + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + (wm * TM + i) * 32 + (r / 4) * 8 + lh * 4 + (r % 4);
        if (row < g.m && col < g.n) {
          float* p = out + int64_t(row) * ld + col;
          const float v = acc[i][j][r];
          if (acc_out) *p = *p + v;
          else if (bias) *p = lin_epi(v, bias[col], g.relu);
          else *p = v;
        }
      }
    }
  }
}

template <int NT, int MINB, class C, bool TA, bool TB>
__global__ __launch_bounds__(NT, MINB) void gemm_f32_lds(GemmArgs g) {
  static_assert(NT == C::THREADS, "one lane per thread of the configuration");
  __shared__ __attribute__((aligned(1024))) float smem[C::STAGES * C::STAGE];
  gemm_f32_lds_tile<C, TA, TB>(g, int(blockIdx.x), int(blockIdx.z), gridDim.z > 1, smem);
}

// Two independent products in one launch (a Linear's weight gradient A and
// input gradient B): workgroups [0, tiles_a * splits_a) compute product A in
// the order of its own launch (split-major, as blockIdx.z then x), the rest
// product B, so every tile and partial holds the bits the product's own
// launch gives.  The CUs product A frees start B's first loads while A's last
// stores drain, where two launches would drain and refill one after the other.
template <int NT, int MINB, class CA, bool TAA, bool TBA, class CB, bool TAB, bool TBB>
__global__ __launch_bounds__(NT, MINB) void gemm_f32_lds_pair(GemmArgs ga, int splits_a,
                                                              GemmArgs gb, int splits_b) {
  static_assert(NT == CA::THREADS && NT == CB::THREADS, "one workgroup size for both");
  constexpr int FA = CA::STAGES * CA::STAGE, FB = CB::STAGES * CB::STAGE;
  __shared__ __attribute__((aligned(1024))) float smem[FA > FB ? FA : FB];
  const int tiles_a = ga.tiles_m * ga.tiles_n, tiles_b = gb.tiles_m * gb.tiles_n;
  const int i = int(blockIdx.x);
  if (i < tiles_a * splits_a) {
    gemm_f32_lds_tile<CA, TAA, TBA>(ga, i % tiles_a, i / tiles_a, splits_a > 1, smem);
  } else {
    const int j = i - tiles_a * splits_a;
    gemm_f32_lds_tile<CB, TAB, TBB>(gb, j % tiles_b, j / tiles_b, splits_b > 1, smem);
  }
}

// ------------------------------------------------------------------ rows
//
// M <= 32 with B transposed and enough columns to give every CU a block of
// 32 (Linear's input gradient dY * W^T at a small batch: C[m, n] =
// sum_k A[m, k] * Bs[n, k] with the weight stored as Bs [n, k]).  Column j of
// C needs row j of Bs in full, so a workgroup that owns 32 columns reads 32
// whole rows of Bs -- one contiguous span of memory -- over all of K: no
// split of K, no partials, no fold.  (The split-K direct kernel instead reads
// 4 KiB pieces of 128 rows 16 KiB apart.)  Its four waves take consecutive
// quarters of K and add their 32x32 blocks through LDS in wave order.
//
// Operands move through wave-private LDS rings: per group of 32 k values a
// 32 x 32 tile of A and one of Bs (4 KiB each), each filled by four
// global_load_lds_dwordx4 instructions whose lanes cover 8 rows x 128 bytes,
// so every instruction reads whole lines (loading straight into MFMA layout
// would spread each instruction over 32 rows).  In LDS a tile row is 128
// bytes and its 16-byte chunk c sits in slot c ^ (row & 7), which the DMA
// arranges by choosing the chunk each lane fetches; fragment reads of a
// wave's 32 rows then spread over the banks.  Lane l holds row l % 32 and,
// in half h = l / 32, k0 + 16 h .. k0 + 16 h + 15 (four 128-bit LDS reads per
// operand); MFMA step s pairs k0 + s with k0 + 16 + s.  STAGES tiles of each
// wave are in flight; rows outside the matrix and k past the wave's range
// read the zero page.
//
// Each workgroup walks its waves' tiles starting at tile (13 * block) mod
// count and wrapping around.  With every workgroup starting at k = 0 the
// whole chip would request the same column offsets of rows 16 KiB apart at
// once, which crowds a few HBM channels (32.6 us for config 3's dX on
// MI355X); staggered starts spread the requests (27.0 us).  The order of the
// k terms then depends on the column block, and is the same on every run.
struct RowsArgs {
  const float* a;
  const float* b;  // stored [n, k]
  float* c;
  int m, n, k;
  int lda, ldb, ldc;
  int accumulate;
  const float* bias;  // per-column bias added to the output (or null)
  int relu;           // with a bias: ReLU after it
  int vec_out;        // C and the bias take 128-bit accesses
};

constexpr int kRowsWaves = 4;
constexpr int kRowsStages = 3;
constexpr int kRowsTile = 32 * 32;  // floats of one operand tile

template <int STAGES>
__global__ __launch_bounds__(64 * kRowsWaves, 1) void gemm_thin_rows(RowsArgs g) {
  constexpr int STAGE = 2 * kRowsTile;  // A tile, then B tile
  __shared__ __attribute__((aligned(1024))) float smem[kRowsWaves * STAGES * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int li = lane & 31, lh = lane >> 5;
  const int n0 = int(blockIdx.x) * 32;
  const int part = ((g.k + kRowsWaves - 1) / kRowsWaves + 31) / 32 * 32;
  const int kb = wave * part;
  const int ke = min(g.k, kb + part);
  const int ntiles = kb < ke ? (ke - kb + 31) / 32 : 0;
  const int rot = ntiles ? int((blockIdx.x * 13u) % uint32_t(ntiles)) : 0;
  float* ring = smem + wave * STAGES * STAGE;
  // The zero page's address, materialised once outside the loop.
  uint64_t zero_bits = reinterpret_cast<uint64_t>(g_direct_zeros);
  asm volatile("" : "+s"(zero_bits));
  const float* zero = reinterpret_cast<const float*>(zero_bits);

  // DMA roles: instruction q of a tile covers rows 8q .. 8q + 7; lane L fills
  // slot (row 8q + L / 8, L % 8), i.e. fetches chunk (L % 8) ^ (row & 7).
  const float* asrc[4];
  const float* bsrc[4];
  int dk[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 8 * q + (lane >> 3);
    const int c = (lane & 7) ^ (row & 7);
    dk[q] = 4 * c;
    asrc[q] = row < g.m ? g.a + int64_t(row) * g.lda + 4 * c : nullptr;
    bsrc[q] = n0 + row < g.n ? g.b + int64_t(n0 + row) * g.ldb + 4 * c : nullptr;
  }
  auto issue = [&](int t) {
    const int tt = t + rot < ntiles ? t + rot : t + rot - ntiles;
    const int k0 = kb + 32 * tt;
    float* st = ring + (t % STAGES) * STAGE;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      lds_dma16(asrc[q] && k0 + dk[q] < ke ? asrc[q] + k0 : zero, st + q * 256);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      lds_dma16_nt(bsrc[q] && k0 + dk[q] < ke ? bsrc[q] + k0 : zero, st + kRowsTile + q * 256);
  };

  v16f acc = v16f(0.0f);
#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t)
    if (t < ntiles) issue(t);
  for (int t = 0; t < ntiles; ++t) {
    // The slot refilled here was read in the previous iteration, whose LDS
    // reads completed before its MFMAs.
    if (t + STAGES - 1 < ntiles) {
      issue(t + STAGES - 1);
      wait_vmcnt<(STAGES - 1) * 8>();  // tile t has landed
    } else {
      wait_vmcnt<0>();
    }
    const float* sa = ring + (t % STAGES) * STAGE;
    const float* sb = sa + kRowsTile;
    v4f fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int slot = li * 32 + (((4 * lh + i) ^ (li & 7)) << 2);
      fa[i] = *reinterpret_cast<const v4f*>(sa + slot);
      fb[i] = *reinterpret_cast<const v4f*>(sb + slot);
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[s / 4][s % 4], fb[s / 4][s % 4], acc, 0, 0, 0);
  }

  // Waves' blocks [wave][r][lane] in LDS (over the rings, once every wave is
  // done with them), summed in wave order.  Thread t owns row t / 8 of the
  // block and its columns 4 (t % 8) .. 4 (t % 8) + 3; accumulator register r
  // of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
  __syncthreads();
  float* red = smem;
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
  __syncthreads();
  const int t = int(threadIdx.x);
  const int row = t >> 3, c4 = (t & 7) * 4;
  const int r = ((row >> 3) << 2) | (row & 3), lhr = (row >> 2) & 1;
  v4f v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int ln = c4 + q + 32 * lhr;
    float s = red[r * 64 + ln];
#pragma unroll
    for (int w = 1; w < kRowsWaves; ++w) s += red[(w * 16 + r) * 64 + ln];
    v[q] = s;
  }
  if (row >= g.m) return;
  float* out = g.c + int64_t(row) * g.ldc;
  const int col = n0 + c4;
  if (g.vec_out) {
    if (col < g.n) {
      v4f* o = reinterpret_cast<v4f*>(out + col);
      if (g.accumulate) *o = *o + v;
      else if (g.bias) *o = lin_epi4(v, *reinterpret_cast<const v4f*>(g.bias + col), g.relu);
      else *o = v;
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (col + q < g.n) {
      float* o = out + col + q;
      if (g.accumulate) *o = *o + v[q];
      else *o = g.bias ? lin_epi(v[q], g.bias[col + q], g.relu) : v[q];
    }
  }
}

// ------------------------------------------------------------ short K
//
// C[m, n] (+)= sum_k A[k, m] * B[k, n] with K <= 32 (A stored [k, m]): the
// weight gradient X^T dY of a Linear at a small batch, a 128 MiB C for a few
// GFLOP.  The 128 x 128 LDS-tile kernel runs each tile as load -> MFMA ->
// store with a workgroup per tile, and measured no faster with more
// workgroups per CU.  Here 2 x CU workgroups stay resident and walk the tiles
// (n fastest, so the workgroups in flight write whole rows of C): each prefetches its
// next tile's panels into the other of two LDS stages before running the
// current tile's MFMAs and stores, so one tile's loads are in flight while
// the previous tile's C leaves.  Panels, swizzle, MFMA step order and the
// column sums (first tile row only, k rows in order within two halves, then
// the halves in order) are those of gemm_f32_lds<LdsSmall> with A transposed,
// so both kernels give identical bits.  The C tile leaves through a
// wave-private 32 x 36 LDS tile inside the stage just consumed.
constexpr int kShortBM = 128, kShortBN = 128;

__global__ __launch_bounds__(256, 2) void gemm_tn_short(GemmArgs g) {
  constexpr int BM = kShortBM, BN = kShortBN, NW = 4, TM = 2, TN = 2;
  constexpr int A_PANEL = BM * kBK, STAGE = (BM + BN) * kBK;  // floats
  constexpr int A_DMA = BM * 8 / 64 / NW, B_DMA = BN * 8 / 64 / NW;
  constexpr int CS_ROWS = kBK / 2;  // two halves of the k rows per column
  __shared__ __attribute__((aligned(1024))) float smem[2 * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int wm = wave / 2, wn = wave % 2;
  const int li = lane & 31, lh = lane >> 5;
  const int ntiles = g.tiles_m * g.tiles_n;
  uint64_t zero_bits = reinterpret_cast<uint64_t>(g_direct_zeros);
  asm volatile("" : "+s"(zero_bits));
  const float* zero = reinterpret_cast<const float*>(zero_bits);

  // DMA roles (N-major panels: k row kr, 16-byte chunk c ^ 8 (kr / 16)).
  int a_kr[A_DMA], a_c[A_DMA], b_kr[B_DMA], b_c[B_DMA];
#pragma unroll
  for (int q = 0; q < A_DMA; ++q) {
    const int p = (wave * A_DMA + q) * 64 + lane;
    a_kr[q] = p / (BM / 4);
    a_c[q] = 4 * ((p % (BM / 4)) ^ ((a_kr[q] >> 4) << 3));
  }
#pragma unroll
  for (int q = 0; q < B_DMA; ++q) {
    const int p = (wave * B_DMA + q) * 64 + lane;
    b_kr[q] = p / (BN / 4);
    b_c[q] = 4 * ((p % (BN / 4)) ^ ((b_kr[q] >> 4) << 3));
  }
  auto issue = [&](int t, int stage) {
    const int m0 = (t / g.tiles_n) * BM, n0 = (t % g.tiles_n) * BN;
    float* sa = smem + stage * STAGE;
    float* sb = sa + A_PANEL;
#pragma unroll
    for (int q = 0; q < A_DMA; ++q) {
      const bool ok = m0 + a_c[q] < g.m && a_kr[q] < g.k;
      lds_dma16(ok ? g.a + int64_t(a_kr[q]) * g.lda + m0 + a_c[q] : zero,
                sa + (wave * A_DMA + q) * 256);
    }
#pragma unroll
    for (int q = 0; q < B_DMA; ++q) {
      const bool ok = n0 + b_c[q] < g.n && b_kr[q] < g.k;
      lds_dma16(ok ? g.b + int64_t(b_kr[q]) * g.ldb + n0 + b_c[q] : zero,
                sb + (wave * B_DMA + q) * 256);
    }
  };

  // Tile (row-major index) at walk position i of this workgroup, or -1 past
  // the end.  Plain walk: tiles blockIdx.x + i * gridDim.x.  XCD-blocked walk
  // (walk_a x walk_b > 0, gridDim.x a multiple of 8, the tile grid split into
  // walk_a x walk_b equal blocks): workgroup b takes block b % 8 (workgroups
  // reach the eight XCDs round-robin), walking it row-major from b / 8 in
  // steps of gridDim.x / 8, so each XCD's L2 sees one block's A and B panels
  // rather than every row of A.  Either way every tile is taken exactly once.
  auto tile_at = [&](int i) -> int {
    if (g.walk_a == 0) {
      const int t = int(blockIdx.x) + i * int(gridDim.x);
      return t < ntiles ? t : -1;
    }
    const int bm = g.tiles_m / g.walk_a, bn = g.tiles_n / g.walk_b;
    const int x = int(blockIdx.x) % 8;
    const int l = int(blockIdx.x) / 8 + i * (int(gridDim.x) / 8);
    if (l >= bm * bn) return -1;
    const int row = (x / g.walk_b) * bm + l / bn, col = (x % g.walk_b) * bn + l % bn;
    return row * g.tiles_n + col;
  };
  int t = tile_at(0);
  if (t >= 0) issue(t, 0);
  for (int it = 0; t >= 0; ++it) {
    const int stage = it & 1;
    const int m0 = (t / g.tiles_n) * BM, n0 = (t % g.tiles_n) * BN;
    // This tile's panels have landed (and the previous tile's stores have
    // been accepted); every wave is past the previous tile's epilogue, which
    // used the other stage, so it may be refilled.
    wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");
    const int t_next = tile_at(it + 1);
    if (t_next >= 0) issue(t_next, stage ^ 1);

    const float* sa = smem + stage * STAGE;
    const float* sb = sa + A_PANEL;
    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = v16f(0.0f);
    // MFMA step s pairs k = s (lanes 0-31) with k = s + 16 (lanes 32-63).
#pragma unroll
    for (int s = 0; s < kBK / 2; ++s) {
      const int kr = lh * (kBK / 2) + s;
      float fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = sa[kr * BM + (((wm * TM + i) * 32 + li) ^ (lh << 5))];
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = sb[kr * BN + (((wn * TN + j) * 32 + li) ^ (lh << 5))];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    // Column sums of B beside the first tile row: thread t owns column t % BN
    // and k rows (t / BN) * 16 .. + 15.
    const bool do_cs = g.colsum != nullptr && m0 == 0;
    float cs = 0.0f;
    if (do_cs) {
      const int col = int(threadIdx.x) % BN, part = int(threadIdx.x) / BN;
#pragma unroll
      for (int r = 0; r < CS_ROWS; ++r) {
        const int kr = part * CS_ROWS + r;
        cs += sb[kr * BN + (col ^ ((kr >> 4) << 5))];
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");  // every wave is done reading this stage

    float* region = smem + stage * STAGE;
    if (do_cs) {
      region[NW * 32 * 36 + threadIdx.x] = cs;
      __syncthreads();
      if (int(threadIdx.x) < BN) {
        const float v = region[NW * 32 * 36 + threadIdx.x] + region[NW * 32 * 36 + BN + threadIdx.x];
        const int col = n0 + int(threadIdx.x);
        if (col < g.n) g.colsum[col] = g.colsum_acc ? g.colsum[col] + v : v;
      }
    }
    float* tile = region + wave * (32 * 36);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          tile[((r / 4) * 8 + lh * 4 + (r % 4)) * 36 + li] = acc[i][j][r];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int row0 = m0 + (wm * TM + i) * 32, col0 = n0 + (wn * TN + j) * 32;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int idx = lane + 64 * q;
          const int rr = idx >> 3, cc = (idx & 7) * 4;
          const v4f v = *reinterpret_cast<const v4f*>(tile + rr * 36 + cc);
          const int row = row0 + rr, col = col0 + cc;
          if (row < g.m && col < g.n) {
            v4f* p = reinterpret_cast<v4f*>(g.c + int64_t(row) * g.ldc + col);
            if (g.accumulate) *p = *p + v;
            else if (g.bias) *p = lin_epi4(v, *reinterpret_cast<const v4f*>(g.bias + col), g.relu);
            else *p = v;
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
    }
    t = t_next;
  }
}

// Default split of K: none once there is a tile for every CU; otherwise
// enough splits to give each CU two workgroups, keeping at least four K tiles
// per split.
int default_splits(Runtime* rt, int tiles, int k_tiles) {
  if (tiles >= rt->cu_count || k_tiles < 8) return 1;
  const int want = 2 * rt->cu_count;
  const int splits = std::min((want + tiles - 1) / tiles, std::max(1, k_tiles / 4));
  return std::max(1, std::min(splits, 64));
}

// Sets g's tile counts for BM x BN tiles and its K tiles per split for a
// requested split count (0: default_splits); returns the split count that
// results, no split left empty.
int set_split(Runtime* rt, GemmArgs& g, int bm, int bn, int splits) {
  g.tiles_m = (g.m + bm - 1) / bm;
  g.tiles_n = (g.n + bn - 1) / bn;
  const int k_tiles = (g.k + kBK - 1) / kBK;
  if (splits <= 0) splits = default_splits(rt, g.tiles_m * g.tiles_n, k_tiles);
  splits = std::max(1, std::min(splits, k_tiles));
  g.k_tiles_per_split = (k_tiles + splits - 1) / splits;
  return std::max(1, (k_tiles + g.k_tiles_per_split - 1) / g.k_tiles_per_split);
}

// The split of the one-workgroup-per-CU LDS configurations: K split so the
// tiles cover the CUs once, keeping at least eight K tiles per split.
template <class L>
int set_split_lds(Runtime* rt, GemmArgs& g) {
  const int tiles = ((g.m + L::BM - 1) / L::BM) * ((g.n + L::BN - 1) / L::BN);
  const int k_tiles = (g.k + kBK - 1) / kBK;
  return set_split(rt, g, L::BM, L::BN, std::max(1, std::min(rt->cu_count / tiles, k_tiles / 8)));
}

template <class C, bool TA, bool TB>
int launch_gemm_cfg(Runtime* rt, GemmArgs g, bool vec, const Workspace& ws, int splits = 0,
                    bool* colsum_done = nullptr) {
  splits = set_split(rt, g, C::BM, C::BN, splits);
  const int tiles = g.tiles_m * g.tiles_n;

  // Column sums ride only on the LDS tiles with B untransposed and no split.
  if (g.colsum && (!(vec && std::is_same_v<C, CfgLarge>) || splits > 1 || TB)) g.colsum = nullptr;
  if (g.colsum && colsum_done) *colsum_done = true;
  float* final_c = g.c;
  float* part = nullptr;
  if (splits > 1) {
    const int wrc = ws.take(size_t(splits) * size_t(g.m) * size_t(g.n) * sizeof(float), &part);
    if (wrc != LMP_OK) return wrc;
    g.c = part;
  }
  const dim3 grid{uint32_t(tiles), 1u, uint32_t(splits)};
  if (vec && std::is_same_v<C, CfgLarge>)
    hipLaunchKernelGGL((gemm_f32_lds<LdsSmall::THREADS, LdsSmall::MINB, LdsSmall, TA, TB>), grid,
                       dim3(LdsSmall::THREADS), 0, rt->stream, g);
  else if (vec)
    hipLaunchKernelGGL((gemm_f32_mfma<C, TA, TB, true>), grid, dim3(kThreads), 0,
                       rt->stream, g);
  else
    hipLaunchKernelGGL((gemm_f32_mfma<C, TA, TB, false>), grid, dim3(kThreads), 0,
                       rt->stream, g);
  LMP_LAUNCH_CHECK("gemm_f32_mfma");
  if (splits > 1) {
    const int frc = launch_fold(rt, final_c, part, g.m, g.n, g.ldc, splits, g.accumulate,
                                g.bias, g.relu);
    ws.give(part);  // stream-ordered: the fold reads it first
    if (frc != LMP_OK) return frc;
  }
  return LMP_OK;
}

// One of the one-workgroup-per-CU LDS configurations (split by set_split_lds).
template <class L, bool TA, bool TB>
int launch_lds(Runtime* rt, GemmArgs g, const Workspace& ws, bool* colsum_done = nullptr) {
  const int splits = set_split_lds<L>(rt, g);
  const int tiles = g.tiles_m * g.tiles_n;
  // Column sums ride only with B untransposed and no split.
  if (g.colsum && (splits > 1 || TB)) g.colsum = nullptr;
  if (g.colsum && colsum_done) *colsum_done = true;
  float* final_c = g.c;
  float* part = nullptr;
  if (splits > 1) {
    const int wrc = ws.take(size_t(splits) * size_t(g.m) * size_t(g.n) * sizeof(float), &part);
    if (wrc != LMP_OK) return wrc;
    g.c = part;
  }
  const dim3 grid{uint32_t(tiles), 1u, uint32_t(splits)};
  hipLaunchKernelGGL((gemm_f32_lds<L::THREADS, L::MINB, L, TA, TB>), grid, dim3(L::THREADS), 0,
                     rt->stream, g);
  LMP_LAUNCH_CHECK("gemm_f32_lds");
  if (splits > 1) {
    const int frc = launch_fold(rt, final_c, part, g.m, g.n, g.ldc, splits, g.accumulate,
                                g.bias, g.relu);
    ws.give(part);  // stream-ordered: the fold reads it first
    if (frc != LMP_OK) return frc;
  }
  return LMP_OK;
}

// M <= 32 on the register-direct kernel.  Each workgroup takes at least 64
// values of k per wave; the split count aims at one workgroup per CU (more
// only adds partial traffic: measured on MI355X); `splits` > 0 overrides it.
template <bool TA, bool TB, int STAGES = 2>
int launch_direct(Runtime* rt, const GemmArgs& g0, const Workspace& ws, int splits = 0) {
  DirectArgs d{};
  d.a = g0.a;
  d.b = g0.b;
  d.c = g0.c;
  d.m = g0.m;
  d.n = g0.n;
  d.k = g0.k;
  d.lda = g0.lda;
  d.ldb = g0.ldb;
  d.ldc = g0.ldc;
  d.accumulate = g0.accumulate;
  d.bias = g0.bias;
  d.relu = g0.relu;
  d.n_blocks = (g0.n + kDirectN - 1) / kDirectN;
  constexpr int kGrain = 8 * kDirectWaves;
  const int max_splits = std::max(1, g0.k / (64 * kDirectWaves));
  if (splits <= 0) splits = (rt->cu_count + d.n_blocks - 1) / d.n_blocks;
  splits = std::max(1, std::min(splits, max_splits));
  d.k_per_wg = ((g0.k + splits - 1) / splits + kGrain - 1) / kGrain * kGrain;
  splits = (g0.k + d.k_per_wg - 1) / d.k_per_wg;
  float* part = nullptr;
  if (splits > 1) {
    const int wrc = ws.take(size_t(splits) * size_t(g0.m) * size_t(g0.n) * sizeof(float), &part);
    if (wrc != LMP_OK) return wrc;
    d.c = part;
  }
  const dim3 grid{uint32_t(d.n_blocks), uint32_t(splits), 1u};
  hipLaunchKernelGGL((gemm_direct<TA, TB, STAGES>), grid, dim3(64 * kDirectWaves), 0, rt->stream,
                     d);
  LMP_LAUNCH_CHECK("gemm_direct");
  if (splits > 1) {
    // The splits of a column block ran on one XCD when the block count is a
    // multiple of eight (workgroups reach the XCDs round-robin).
    const int cb = d.n_blocks % 8 == 0 && kDirectN == 128 ? d.n_blocks : 0;
    const int frc = launch_fold(rt, g0.c, part, g0.m, g0.n, g0.ldc, splits, g0.accumulate,
                                g0.bias, g0.relu, cb);
    ws.give(part);  // stream-ordered: the fold reads it first
    if (frc != LMP_OK) return frc;
  }
  return LMP_OK;
}

// K <= 32 with A transposed on the persistent short-K kernel: two resident
// workgroups per CU walk the 128 x 128 tiles.
int launch_short(Runtime* rt, GemmArgs g, bool* colsum_done) {
  g.tiles_m = (g.m + kShortBM - 1) / kShortBM;
  g.tiles_n = (g.n + kShortBN - 1) / kShortBN;
  const int64_t tiles = int64_t(g.tiles_m) * g.tiles_n;
  if (g.colsum && colsum_done) *colsum_done = true;
  const uint32_t grid = uint32_t(std::min<int64_t>(tiles, 2 * int64_t(rt->cu_count)));
  // XCD-blocked walk when the tiles split into eight equal blocks: the block
  // shape that gives each XCD the fewest A and B panels to read.
  g.walk_a = g.walk_b = 0;
  if (grid % 8 == 0) {
    int64_t best = 0;
    for (int a = 1; a <= 8; a *= 2) {
      const int b = 8 / a;
      if (g.tiles_m % a != 0 || g.tiles_n % b != 0) continue;
      const int64_t panels = int64_t(g.tiles_m / a) * kShortBM + int64_t(g.tiles_n / b) * kShortBN;
      if (best == 0 || panels < best) {
        best = panels;
        g.walk_a = a;
        g.walk_b = b;
      }
    }
  }
  hipLaunchKernelGGL(gemm_tn_short, dim3(grid), dim3(256), 0, rt->stream, g);
  LMP_LAUNCH_CHECK("gemm_tn_short");
  return LMP_OK;
}

// M <= 32 with B transposed on the whole-rows kernel: one workgroup per 32
// columns, no split of K.
int launch_rows(Runtime* rt, const GemmArgs& g0) {
  RowsArgs r{};
  r.a = g0.a;
  r.b = g0.b;
  r.c = g0.c;
  r.m = g0.m;
  r.n = g0.n;
  r.k = g0.k;
  r.lda = g0.lda;
  r.ldb = g0.ldb;
  r.ldc = g0.ldc;
  r.accumulate = g0.accumulate;
  r.bias = g0.bias;
  r.relu = g0.relu;
  r.vec_out = g0.vec_out;
  const dim3 grid{uint32_t((g0.n + 31) / 32), 1u, 1u};
  hipLaunchKernelGGL(gemm_thin_rows<kRowsStages>, grid, dim3(64 * kRowsWaves), 0, rt->stream, r);
  LMP_LAUNCH_CHECK("gemm_thin_rows");
  return LMP_OK;
}

// Kernel choice (measured on MI355X, fp32), in order: the tiny kernel for
// small latency-bound products (K <= 512, at most 2^21 multiply-adds); the
// persistent short-K kernel (A transposed, K <= 32); whole rows of B per
// workgroup (M <= 32, B transposed, a 32-column block per CU); the
// register-direct kernel (M <= 32) and 32 x 256 tiles (M <= 64); then, with
// 16-byte operand rows, the LDS-DMA configurations (256 x 256 when they cover
// the CUs, 256 x 128 split for M >= 512, N >= 2048, K >= 2048, 128 x 64 split
// when 128 x 128 tiles would not cover the CUs); otherwise 64 x 64 register
// tiles without a split for a short K (<= 2048) with too few 128 x 128 tiles,
// else 128 x 128 (on LDS-DMA tiles when the rows allow) with split K.  Single
// and paired launches take their kernel from this one function.
enum class Route { Tiny, Short, Rows, Direct, Skinny, Big, Wide, Mid, Small64, Large };

template <bool TA, bool TB>
Route gemm_route(Runtime* rt, const GemmArgs& g, bool vec, bool direct_ok) {
  if (tiny_ok(g)) return Route::Tiny;
  // K <= 32 with A transposed (a Linear's weight gradient at a small batch):
  // the persistent short-K kernel, whose tiles and orders are those of the
  // 128 x 128 LDS tiles it replaces here.
  if constexpr (TA && !TB) {
    const int64_t short_tiles = int64_t((g.m + kShortBM - 1) / kShortBM) *
                                ((g.n + kShortBN - 1) / kShortBN);
    if (vec && g.vec_out && g.k <= kBK && short_tiles <= 0x7fffffff)
      return Route::Short;
  }
  // M <= 32 with B transposed and a 32-column block for every CU: whole rows
  // of B per workgroup, no split (config 3's dX: 46 -> 31-35 us cold).
  if constexpr (!TA && TB) {
    if (direct_ok && g.m <= 32 && (g.n + 31) / 32 >= rt->cu_count) return Route::Rows;
  }
  if (direct_ok && g.m <= 32) return Route::Direct;
  if (g.m <= 64) return Route::Skinny;
  if (vec) {
    const int64_t big_tiles = int64_t((g.m + LdsBig::BM - 1) / LdsBig::BM) *
                              ((g.n + LdsBig::BN - 1) / LdsBig::BN);
    // (K of a few tiles leaves the kernel bound by writing C: more, smaller
    // tiles do better there.)
    if (big_tiles >= rt->cu_count && g.k >= 256) return Route::Big;
    if (g.m >= 512 && g.n >= 2048 && g.k >= 2048) return Route::Wide;
    const int64_t tiles128 = int64_t((g.m + 127) / 128) * ((g.n + 127) / 128);
    if (tiles128 < rt->cu_count && g.k >= 512) return Route::Mid;
  }
  const int64_t large_tiles = int64_t((g.m + CfgLarge::BM - 1) / CfgLarge::BM) *
                              ((g.n + CfgLarge::BN - 1) / CfgLarge::BN);
  const int64_t small_tiles = int64_t((g.m + CfgSmall::BM - 1) / CfgSmall::BM) *
                              ((g.n + CfgSmall::BN - 1) / CfgSmall::BN);
  if (large_tiles < rt->cu_count && g.k <= 2048 && small_tiles >= rt->cu_count)
    return Route::Small64;
  return Route::Large;
}

template <bool TA, bool TB>
int launch_gemm(Runtime* rt, const GemmArgs& g, bool vec, bool direct_ok, const Workspace& ws,
                bool* colsum_done = nullptr) {
  switch (gemm_route<TA, TB>(rt, g, vec, direct_ok)) {
    case Route::Tiny:
      if (g.colsum && colsum_done) *colsum_done = true;
      return launch_tiny<TA, TB>(rt, g);
    case Route::Short: return launch_short(rt, g, colsum_done);
    case Route::Rows: return launch_rows(rt, g);
    // With B transposed a wave's loads touch more cache lines per byte, so
    // three fragments in flight instead of two.
    case Route::Direct: return launch_direct<TA, TB, TB ? 3 : 2>(rt, g, ws);
    case Route::Skinny: return launch_gemm_cfg<CfgSkinny, TA, TB>(rt, g, vec, ws);
    case Route::Big: return launch_lds<LdsBig, TA, TB>(rt, g, ws, colsum_done);
    case Route::Wide: return launch_lds<LdsWide, TA, TB>(rt, g, ws, colsum_done);
    case Route::Mid: return launch_lds<LdsMid, TA, TB>(rt, g, ws, colsum_done);
    case Route::Small64: return launch_gemm_cfg<CfgSmall, TA, TB>(rt, g, vec, ws, 1);
    case Route::Large: return launch_gemm_cfg<CfgLarge, TA, TB>(rt, g, vec, ws, 0, colsum_done);
  }
  return fail(LMP_ERR_RUNTIME, "gemm: no kernel for this product");
}

// ------------------------------------------------------ weight + input pair

// The LDS configuration a product's own launch would use, with its tiles and
// split set in g: 0 (not an LDS-tile launch), else the configuration's id
// (1 Big, 2 Wide, 3 Mid, 4 the 128 x 128 LDS tiles of the Large route).
template <bool TA, bool TB>
int lds_config_of(Runtime* rt, GemmArgs& g, bool vec, bool direct_ok, int* splits) {
  switch (gemm_route<TA, TB>(rt, g, vec, direct_ok)) {
    case Route::Big: *splits = set_split_lds<LdsBig>(rt, g); return 1;
    case Route::Wide: *splits = set_split_lds<LdsWide>(rt, g); return 2;
    case Route::Mid: *splits = set_split_lds<LdsMid>(rt, g); return 3;
    case Route::Large:
      if (!vec) return 0;
      *splits = set_split(rt, g, CfgLarge::BM, CfgLarge::BN, 0);
      return 4;
    default: return 0;
  }
}

template <class CW, class CX>
int launch_pair(Runtime* rt, GemmArgs gw, int sw, GemmArgs gx, int sx) {
  static_assert(CW::THREADS == CX::THREADS, "one workgroup size for both");
  const Workspace ws{};
  float* pw = nullptr;
  float* px = nullptr;
  float* const cw = gw.c;
  float* const cx = gx.c;
  if (sw > 1) {
    const int rc = ws.take(size_t(sw) * size_t(gw.m) * size_t(gw.n) * sizeof(float), &pw);
    if (rc != LMP_OK) return rc;
    gw.c = pw;
  }
  if (sx > 1) {
    const int rc = ws.take(size_t(sx) * size_t(gx.m) * size_t(gx.n) * sizeof(float), &px);
    if (rc != LMP_OK) {
      if (pw) ws.give(pw);
      return rc;
    }
    gx.c = px;
  }
  constexpr int kMinB = CW::MINB > CX::MINB ? CW::MINB : CX::MINB;
  const int64_t wgs = int64_t(gw.tiles_m) * gw.tiles_n * sw + int64_t(gx.tiles_m) * gx.tiles_n * sx;
  hipLaunchKernelGGL((gemm_f32_lds_pair<CW::THREADS, kMinB, CW, true, false, CX, false, true>),
                     dim3(uint32_t(wgs)), dim3(CW::THREADS), 0, rt->stream, gw, sw, gx, sx);
  LMP_LAUNCH_CHECK("gemm_f32_lds_pair");
  int rc = LMP_OK;
  if (sw > 1) rc = launch_fold(rt, cw, pw, gw.m, gw.n, gw.ldc, sw, gw.accumulate, nullptr, 0);
  if (rc == LMP_OK && sx > 1)
    rc = launch_fold(rt, cx, px, gx.m, gx.n, gx.ldc, sx, gx.accumulate, nullptr, 0);
  if (pw) ws.give(pw);  // stream-ordered: the folds read them first
  if (px) ws.give(px);
  return rc;
}

// dW = X^T G (with db, the column sums of G, when gw.colsum is set) and
// dX = G W^T in one launch when both take LDS tiles of one workgroup size,
// each with the configuration and split of its own launch (so the same bits
// as lmp_k_gemm_colsum_f32 and lmp_k_gemm_f32); the column sums must then ride
// in the dW tiles (dW unsplit).  Returns false, with nothing launched, when
// the pair does not apply.
bool try_linear_backward_pair(Runtime* rt, GemmArgs gw, bool vec_w, bool direct_w, GemmArgs gx,
                              bool vec_x, bool direct_x, int* rc) {
  int sw = 1, sx = 1;
  const int kw = lds_config_of<true, false>(rt, gw, vec_w, direct_w, &sw);
  const int kx = lds_config_of<false, true>(rt, gx, vec_x, direct_x, &sx);
  if (kw == 0 || kx == 0) return false;
  if (gw.colsum && sw > 1) return false;
  const bool wide_w = kw <= 2, wide_x = kx <= 2;  // 512-thread configurations
  if (wide_w != wide_x) return false;
  switch (kw * 8 + kx) {
    case 1 * 8 + 1: *rc = launch_pair<LdsBig, LdsBig>(rt, gw, sw, gx, sx); return true;
    case 1 * 8 + 2: *rc = launch_pair<LdsBig, LdsWide>(rt, gw, sw, gx, sx); return true;
    case 2 * 8 + 1: *rc = launch_pair<LdsWide, LdsBig>(rt, gw, sw, gx, sx); return true;
    case 2 * 8 + 2: *rc = launch_pair<LdsWide, LdsWide>(rt, gw, sw, gx, sx); return true;
    case 3 * 8 + 3: *rc = launch_pair<LdsMid, LdsMid>(rt, gw, sw, gx, sx); return true;
    case 3 * 8 + 4: *rc = launch_pair<LdsMid, LdsSmall>(rt, gw, sw, gx, sx); return true;
    case 4 * 8 + 3: *rc = launch_pair<LdsSmall, LdsMid>(rt, gw, sw, gx, sx); return true;
    case 4 * 8 + 4: *rc = launch_pair<LdsSmall, LdsSmall>(rt, gw, sw, gx, sx); return true;
    default: return false;
  }
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ------------------------------------------------------ strided column sums

// colsum[j] (+)= sum over r < k of op(B)[r][j], folded in index order, for a B
// whose rows are strided (ldb): the column-sum GEMM's second launch when the
// sums could not ride in the GEMM.  B untransposed ([k, ldb]): one lane per
// column, coalesced row by row.  B transposed (stored [n, ldb]): one wave per
// output, lanes striding over the row, then a butterfly.  256 lanes per
// workgroup; the grid is ceil(n / 256) or ceil(n / 4) workgroups.
__global__ __launch_bounds__(256) void colsum_strided_f32(float* __restrict__ out,
                                                          const float* __restrict__ b, int k,
                                                          int n, int ldb, int trans_b,
                                                          int accumulate) {
  // Indices in 64 bits: the last workgroup's lanes reach past n (and a lane's
  // last step past k), which for extents near 2^31 would not fit an int.
  if (!trans_b) {
    const int64_t j = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (j >= n) return;
    float s = 0.0f;
    for (int64_t r = 0; r < k; ++r) s += b[r * int64_t(ldb) + j];
    out[j] = accumulate ? out[j] + s : s;
    return;
  }
  const int64_t j = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = int(threadIdx.x & 63);
  if (j >= n) return;  // the whole wave leaves together
  const float* row = b + j * int64_t(ldb);
  float s = 0.0f;
  for (int64_t r = lane; r < k; r += 64) s += row[r];
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) out[j] = accumulate ? out[j] + s : s;
}

// ------------------------------------------------------------- transpose

template <typename T>
__global__ __launch_bounds__(256) void transpose_tiled(T* __restrict__ out,
                                                       const T* __restrict__ in,
                                                       int64_t m, int64_t n) {
  __shared__ T tile[64][65];
  const int64_t r0 = int64_t(blockIdx.y) * 64, c0 = int64_t(blockIdx.x) * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
#pragma unroll
  for (int k = 0; k < 64; k += 4) {
    const int64_t r = r0 + ty + k, c = c0 + tx;
    if (r < m && c < n) tile[ty + k][tx] = in[r * n + c];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 64; k += 4) {
    const int64_t r = c0 + ty + k, c = r0 + tx;  // out is [n, m]
    if (r < n && c < m) out[r * m + c] = tile[tx][ty + k];
  }
}

}  // namespace
}  // namespace lmp_hip

using namespace lmp_hip;

namespace {

// Access widths a product allows: g.vec_out (C, and the bias, take 128-bit
// stores), *vec (128-bit panel loads: 16-byte rows and a contiguous extent
// that is a multiple of four), *direct_ok (the register-direct kernel, whose
// float4 C stores need 16-byte C rows when B is untransposed, and a float4
// bias read when there is a bias).
void gemm_flags(GemmArgs& g, int trans_a, int trans_b, bool* vec, bool* direct_ok) {
  g.vec_out = g.n % 4 == 0 && g.ldc % 4 == 0 && aligned16(g.c) && (!g.bias || aligned16(g.bias));
  const int a_contig = trans_a ? g.m : g.k;
  const int b_contig = trans_b ? g.k : g.n;
  *vec = g.lda % 4 == 0 && g.ldb % 4 == 0 && a_contig % 4 == 0 && b_contig % 4 == 0 &&
         aligned16(g.a) && aligned16(g.b);
  *direct_ok = *vec && (trans_b || (g.ldc % 4 == 0 && aligned16(g.c) &&
                                    (!g.bias || aligned16(g.bias))));
}

int gemm_f32_entry(int trans_a, int trans_b, size_t m, size_t n, size_t k,
                   const float* a, size_t lda, const float* b, size_t ldb,
                   const float* bias, float* c, size_t ldc, int accumulate, int relu = 0,
                   const Workspace& ws = Workspace{}, float* colsum = nullptr,
                   int colsum_acc = 0, bool* colsum_done = nullptr) {
  if (m == 0 || n == 0) return LMP_OK;
  if (!c) return fail(LMP_ERR_INVALID, "gemm: null output");
  if (k == 0 && bias)
    return fail(LMP_ERR_UNSUPPORTED, "linear: k == 0");
  if (k == 0) {
    if (accumulate) return LMP_OK;
    if (ldc != n) return fail(LMP_ERR_UNSUPPORTED, "gemm: k == 0 with ldc != n");
    return lmp_k_fill(LMP_FLOAT32, c, m * n, 0.0);
  }
  if (!a || !b) return fail(LMP_ERR_INVALID, "gemm: null input");
  const size_t lim = kGemmMaxExtent - 1;
  if (m > lim || n > lim || k > lim || lda > lim || ldb > lim || ldc > lim)
    return fail(LMP_ERR_UNSUPPORTED, "gemm: dimension of 2^31 - 4096 or more");
  if ((trans_a ? lda < m : lda < k) || (trans_b ? ldb < k : ldb < n) || ldc < n)
    return fail(LMP_ERR_INVALID, "gemm: leading dimension too small");
  LMP_RUNTIME_OR_FAIL(rt);
  // The kernel choice must not depend on the bias (a Linear equals the GEMM
  // followed by the bias add bit for bit only if both run the same kernel),
  // and the kernels read the bias four columns at a time: a bias that is not
  // 16-byte aligned is first copied to one that is.
  float* bias_copy = nullptr;
  if (bias && !aligned16(bias)) {
    bias_copy = static_cast<float*>(scratch_alloc(n * sizeof(float)));
    if (!bias_copy) return LMP_ERR_OOM;
    const hipError_t e = hipMemcpyAsync(bias_copy, bias, n * sizeof(float),
                                        hipMemcpyDeviceToDevice, rt->stream);
    if (e != hipSuccess) {
      scratch_free(bias_copy);
      return fail(LMP_ERR_RUNTIME, std::string("linear: bias copy: ") + hipGetErrorString(e));
    }
    bias = bias_copy;
  }
  GemmArgs g{};
  g.a = a;
  g.b = b;
  g.c = c;
  g.m = int(m);
  g.n = int(n);
  g.k = int(k);
  g.lda = int(lda);
  g.ldb = int(ldb);
  g.ldc = int(ldc);
  g.accumulate = accumulate ? 1 : 0;
  g.bias = bias;
  g.relu = bias && relu ? 1 : 0;
  g.colsum = colsum;
  g.colsum_acc = colsum_acc ? 1 : 0;
  bool vec = false, direct_ok = false;
  gemm_flags(g, trans_a, trans_b, &vec, &direct_ok);
  bool* cd = colsum_done;
  int rc;
  if (!trans_a && !trans_b) rc = launch_gemm<false, false>(rt, g, vec, direct_ok, ws, cd);
  else if (!trans_a && trans_b) rc = launch_gemm<false, true>(rt, g, vec, direct_ok, ws, cd);
  else if (trans_a && !trans_b) rc = launch_gemm<true, false>(rt, g, vec, direct_ok, ws, cd);
  else rc = launch_gemm<true, true>(rt, g, vec, direct_ok, ws, cd);
  if (bias_copy) scratch_free(bias_copy);  // stream-ordered: the kernels read it first
  return rc;
}

}  // namespace

extern "C" int lmp_k_gemm_f32(int trans_a, int trans_b, size_t m, size_t n,
                              size_t k, const float* a, size_t lda,
                              const float* b, size_t ldb, float* c, size_t ldc,
                              int accumulate) {
  return gemm_f32_entry(trans_a, trans_b, m, n, k, a, lda, b, ldb, nullptr, c, ldc,
                        accumulate);
}

extern "C" int lmp_k_gemm_f32_noalloc(int trans_a, int trans_b, size_t m, size_t n,
                                      size_t k, const float* a, size_t lda,
                                      const float* b, size_t ldb, float* c, size_t ldc,
                                      int accumulate) {
  LMP_RUNTIME_OR_FAIL(rt);
  if (!rt->noalloc_scratch)
    return fail(LMP_ERR_RUNTIME, "gemm_noalloc: no workspace on this device (" +
                                     rt->noalloc_error + ")");
  const Workspace ws{static_cast<float*>(rt->noalloc_scratch), LMP_NOALLOC_SCRATCH_BYTES};
  return gemm_f32_entry(trans_a, trans_b, m, n, k, a, lda, b, ldb, nullptr, c, ldc, accumulate,
                        0, ws);
}

extern "C" int lmp_k_linear_f32(int trans_a, int trans_b, size_t m, size_t n,
                                size_t k, const float* a, size_t lda,
                                const float* b, size_t ldb, const float* bias,
                                float* c, size_t ldc) {
  if (!bias) return fail(LMP_ERR_INVALID, "linear: null bias");
  return gemm_f32_entry(trans_a, trans_b, m, n, k, a, lda, b, ldb, bias, c, ldc, 0);
}

extern "C" int lmp_k_gemm_colsum_f32(int trans_a, int trans_b, size_t m, size_t n, size_t k,
                                     const float* a, size_t lda, const float* b, size_t ldb,
                                     float* c, size_t ldc, int accumulate, float* colsum,
                                     int colsum_accumulate) {
  if (!colsum) return fail(LMP_ERR_INVALID, "gemm_colsum: null column-sum output");
  if (m == 0 || n == 0 || k == 0 || !a || !b || !c)
    return fail(LMP_ERR_UNSUPPORTED, "gemm_colsum: empty or null operand");
  const size_t lim = kGemmMaxExtent - 1;
  if (m > lim || n > lim || k > lim || lda > lim || ldb > lim || ldc > lim)
    return fail(LMP_ERR_UNSUPPORTED, "gemm: dimension of 2^31 - 4096 or more");
  if ((trans_a ? lda < m : lda < k) || (trans_b ? ldb < k : ldb < n) || ldc < n)
    return fail(LMP_ERR_INVALID, "gemm: leading dimension too small");
  GemmArgs g{};
  g.a = a;
  g.b = b;
  g.c = c;
  g.m = int(m);
  g.n = int(n);
  g.k = int(k);
  g.lda = int(lda);
  g.ldb = int(ldb);
  g.ldc = int(ldc);
  g.accumulate = accumulate ? 1 : 0;
  g.colsum = colsum;
  g.colsum_acc = colsum_accumulate ? 1 : 0;
  if (tiny_ok(g)) {
    LMP_RUNTIME_OR_FAIL(rt);
    return trans_a ? (trans_b ? launch_tiny<true, true>(rt, g) : launch_tiny<true, false>(rt, g))
                   : (trans_b ? launch_tiny<false, true>(rt, g)
                              : launch_tiny<false, false>(rt, g));
  }
  // Larger products: the column sums ride in the GEMM when it runs on LDS
  // tiles (B untransposed, K unsplit) or on the short-K kernel; otherwise the
  // GEMM, then the column sums of op(B) by the reduction kernels (contiguous
  // B) or by colsum_strided_f32 (strided B).  Everything the second launch
  // needs is reserved before the first, so a refusal leaves C untouched.
  const bool contiguous_b = ldb == (trans_b ? k : n);
  float* dst = colsum;
  if (contiguous_b && colsum_accumulate) {
    dst = static_cast<float*>(scratch_alloc(n * sizeof(float)));
    if (!dst) return LMP_ERR_OOM;
  }
  bool fused = false;
  int rc = gemm_f32_entry(trans_a, trans_b, m, n, k, a, lda, b, ldb, nullptr, c, ldc,
                          accumulate, 0, Workspace{}, colsum, colsum_accumulate, &fused);
  if (rc == LMP_OK && !fused) {
    if (contiguous_b) {
      // sum over k of op(B)[k][j]: B [k, n] reduces over its rows, B^T (stored
      // [n, k]) over its columns.
      const size_t outer = trans_b ? n : 1, len = k, inner = trans_b ? 1 : n;
      rc = lmp_k_reduce(LMP_RED_SUM, LMP_FLOAT32, dst, b, outer, len, inner);
      if (rc == LMP_OK && colsum_accumulate) rc = lmp_k_add_inplace(LMP_FLOAT32, colsum, dst, n);
    } else {
      LMP_RUNTIME_OR_FAIL(rt);
      const uint32_t grid = uint32_t(trans_b ? (n + 3) / 4 : (n + 255) / 256);
      hipLaunchKernelGGL(colsum_strided_f32, dim3(grid), dim3(256), 0, rt->stream, colsum, b,
                         int(k), int(n), int(ldb), trans_b ? 1 : 0, colsum_accumulate ? 1 : 0);
      LMP_LAUNCH_CHECK("colsum_strided_f32");
    }
  }
  if (dst != colsum) scratch_free(dst);  // stream-ordered: the add reads it first
  return rc;
}

extern "C" int lmp_k_gemm_colsum_masked_f32(int trans_a, size_t m, size_t n, size_t k,
                                            const float* a, size_t lda, const float* b,
                                            const float* bmask, size_t ldb, float* c,
                                            size_t ldc, int accumulate, float* colsum,
                                            int colsum_accumulate) {
  if (!colsum || !bmask)
    return fail(LMP_ERR_INVALID, "gemm_colsum_masked: null column sums or mask");
  if (m == 0 || n == 0 || k == 0 || !a || !b || !c)
    return fail(LMP_ERR_UNSUPPORTED, "gemm_colsum_masked: empty or null operand");
  const size_t lim = kGemmMaxExtent - 1;
  if (m > lim || n > lim || k > lim || lda > lim || ldb > lim || ldc > lim)
    return fail(LMP_ERR_UNSUPPORTED, "gemm: dimension of 2^31 - 4096 or more");
  if ((trans_a ? lda < m : lda < k) || ldb < n || ldc < n)
    return fail(LMP_ERR_INVALID, "gemm: leading dimension too small");
  GemmArgs g{};
  g.a = a;
  g.b = b;
  g.c = c;
  g.m = int(m);
  g.n = int(n);
  g.k = int(k);
  g.lda = int(lda);
  g.ldb = int(ldb);
  g.ldc = int(ldc);
  g.accumulate = accumulate ? 1 : 0;
  g.colsum = colsum;
  g.colsum_acc = colsum_accumulate ? 1 : 0;
  g.bmask = bmask;
  if (tiny_ok(g)) {  // the mask applied as B is loaded: one launch
    LMP_RUNTIME_OR_FAIL(rt);
    return trans_a ? launch_tiny<true, false>(rt, g) : launch_tiny<false, false>(rt, g);
  }
  // Larger products: the masked gradient into a contiguous scratch [k, n] by
  // the clamp-backward kernel, then the column-sum GEMM on it.
  float* gm = static_cast<float*>(scratch_alloc(k * n * sizeof(float)));
  if (!gm) return LMP_ERR_OOM;
  lmp_bcast d{};
  d.ndim = 2;
  d.shape[0] = int64_t(k);
  d.shape[1] = int64_t(n);
  d.stride_a[0] = d.stride_b[0] = int64_t(ldb);
  d.stride_a[1] = d.stride_b[1] = 1;
  int rc = lmp_k_binary(LMP_BIN_CLAMP_BACKWARD, LMP_FLOAT32, gm, bmask, b, &d, 0.0,
                        std::numeric_limits<double>::max());
  if (rc == LMP_OK)
    rc = lmp_k_gemm_colsum_f32(trans_a, 0, m, n, k, a, lda, gm, n, c, ldc, accumulate, colsum,
                               colsum_accumulate);
  scratch_free(gm);  // stream-ordered: the GEMM reads it first
  return rc;
}

extern "C" int lmp_k_linear_backward_f32(size_t batch, size_t in, size_t out, const float* x,
                                         size_t ldx, const float* w, size_t ldw, const float* g,
                                         size_t ldg, float* dx, size_t lddx, int dx_accumulate,
                                         float* dw, size_t lddw, int dw_accumulate, float* db,
                                         int db_accumulate) {
  if (!dx || !dw || !db) return fail(LMP_ERR_INVALID, "linear_backward: null output");
  if (batch == 0 || in == 0 || out == 0 || !x || !w || !g)
    return fail(LMP_ERR_UNSUPPORTED, "linear_backward: empty or null operand");
  const size_t lim = kGemmMaxExtent - 1;
  if (batch > lim || in > lim || out > lim || ldx > lim || ldw > lim || ldg > lim ||
      lddx > lim || lddw > lim)
    return fail(LMP_ERR_UNSUPPORTED, "gemm: dimension of 2^31 - 4096 or more");
  if (ldx < in || ldw < out || ldg < out || lddx < in || lddw < out)
    return fail(LMP_ERR_INVALID, "gemm: leading dimension too small");
  // dW [in, out] = X^T G over the batch, with db beside it.
  GemmArgs gw{};
  gw.a = x;
  gw.b = g;
  gw.c = dw;
  gw.m = int(in);
  gw.n = int(out);
  gw.k = int(batch);
  gw.lda = int(ldx);
  gw.ldb = int(ldg);
  gw.ldc = int(lddw);
  gw.accumulate = dw_accumulate ? 1 : 0;
  gw.colsum = db;
  gw.colsum_acc = db_accumulate ? 1 : 0;
  // dX [batch, in] = G W^T over the outputs.
  GemmArgs gx{};
  gx.a = g;
  gx.b = w;
  gx.c = dx;
  gx.m = int(batch);
  gx.n = int(in);
  gx.k = int(out);
  gx.lda = int(ldg);
  gx.ldb = int(ldw);
  gx.ldc = int(lddx);
  gx.accumulate = dx_accumulate ? 1 : 0;
  LMP_RUNTIME_OR_FAIL(rt);
  if (tiny16(rt, gw) && tiny16(rt, gx)) return launch_tiny_linear_backward(rt, gw, gx);
  // Larger products on LDS tiles of one workgroup size: dW (with db) and dX in
  // one launch.
  {
    bool vec_w = false, vec_x = false, direct_w = false, direct_x = false;
    gemm_flags(gw, 1, 0, &vec_w, &direct_w);
    gemm_flags(gx, 0, 1, &vec_x, &direct_x);
    int rc = LMP_OK;
    if (try_linear_backward_pair(rt, gw, vec_w, direct_w, gx, vec_x, direct_x, &rc)) return rc;
  }
  // dW and db first: that call refuses before it launches anything, and dX
  // (a plain GEMM) can then only fail by running out of memory.
  const int rc = lmp_k_gemm_colsum_f32(1, 0, in, out, batch, x, ldx, g, ldg, dw, lddw,
                                       dw_accumulate, db, db_accumulate);
  if (rc != LMP_OK) return rc;
  return lmp_k_gemm_f32(0, 1, batch, in, out, g, ldg, w, ldw, dx, lddx, dx_accumulate);
}

extern "C" int lmp_k_linear_relu_f32(int trans_a, int trans_b, size_t m, size_t n,
                                     size_t k, const float* a, size_t lda,
                                     const float* b, size_t ldb, const float* bias,
                                     float* c, size_t ldc) {
  if (!bias) return fail(LMP_ERR_INVALID, "linear_relu: null bias");
  if (k == 0) return fail(LMP_ERR_UNSUPPORTED, "linear_relu: k == 0");
  return gemm_f32_entry(trans_a, trans_b, m, n, k, a, lda, b, ldb, bias, c, ldc, 0, 1);
}

extern "C" int lmp_k_transpose(int dtype, void* out, const void* in, size_t m,
                               size_t n) {
  if (m == 0 || n == 0) return LMP_OK;
  if (!out || !in) return fail(LMP_ERR_INVALID, "transpose: null buffer");
  LMP_RUNTIME_OR_FAIL(rt);
  const uint64_t gx = (n + 63) / 64, gy = (m + 63) / 64;
  if (gx > 0x7fffffffull || gy > 65535)
    return fail(LMP_ERR_UNSUPPORTED, "transpose: matrix too large");
  const dim3 grid{uint32_t(gx), uint32_t(gy), 1u};
  switch (dtype) {
#define LMP_CASE(CODE, T)                                                     \
  case CODE:                                                                  \
    hipLaunchKernelGGL((transpose_tiled<T>), grid, dim3(256), 0, rt->stream,  \
                       static_cast<T*>(out), static_cast<const T*>(in),       \
                       int64_t(m), int64_t(n));                               \
    LMP_LAUNCH_CHECK("transpose_tiled");                                      \
    return LMP_OK;
    LMP_CASE(LMP_BOOL, bool)
    LMP_CASE(LMP_INT16, int16_t)
    LMP_CASE(LMP_INT32, int32_t)
    LMP_CASE(LMP_INT64, int64_t)
    LMP_CASE(LMP_FLOAT32, float)
    LMP_CASE(LMP_FLOAT64, double)
#undef LMP_CASE
    default:
      return fail(LMP_ERR_INVALID, "transpose: unknown dtype");
  }
}
