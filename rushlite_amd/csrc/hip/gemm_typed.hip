// GEMM for the non-fp32 dtypes: float64 on the matrix cores
// (v_mfma_f64_16x16x4f64) and bool / int16 / int32 / int64 on the vector ALUs.
//
// Lamp3 instantiates its matmul for every dtype (matrix.cu:208-216,
// cpu/matrix.cpp:44-52) with the semantics of cpu/matrix.cpp:8-18: the sum
// starts at 0 in the output type and adds static_cast<Out>(a) *
// static_cast<Out>(b).  For the integer types that is arithmetic modulo 2^bits
// (int16 products are formed in int and truncated when stored back), which
// the kernels reproduce with unsigned accumulators of the output's width so no
// signed overflow occurs; for bool every product is a && b and the sum is an
// OR.  Operands arrive already cast to the output type.
//
// float64 tiling.  A workgroup of 4 waves owns a 64 x 64 tile of C (128 x 128
// once those tiles cover the CUs, gemm_f64_big); each wave
// owns 2 x 2 blocks of 16 x 16 accumulated by v_mfma_f64_16x16x4f64 (lane l
// supplies A[l % 16][l / 16] and B[l / 16][l % 16]; accumulator register r
// holds row 4r + l / 16, column l % 16).  K advances 16 at a time through two
// LDS buffers with register prefetch of the next tile, one barrier per step.
// The integer kernel uses the same 64 x 64 tiles staged through LDS, each
// thread owning a 4 x 4 block of C.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "common.hpp"

namespace lmp_hip {

typedef double v4d __attribute__((ext_vector_type(4)));
typedef double v2d __attribute__((ext_vector_type(2)));

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;
constexpr int kBK = 16;

struct TypedArgs {
  const void* a;
  const void* b;
  void* c;
  int m, n, k;
  int lda, ldb, ldc;
  int accumulate;
  int vec;  // float64: both operands 16-byte aligned with even leading dimensions
};

// Thread f's element of a [kTile x kBK] A tile (row-major in k when !TA) or a
// [kBK x kTile] B tile, loaded so consecutive threads read consecutive
// addresses of the stored matrix.  Returns the tile coordinates (r, c) as
// (m or n index, k index) and the value, zero outside the matrix.
template <typename T, bool TRANS_CONTIG_K>
__device__ __forceinline__ T load_elem(const T* __restrict__ p, int ld, int f, int base,
                                       int k0, int extent, int K, int* idx, int* kk) {
  // TRANS_CONTIG_K: the stored matrix is contiguous along k ([extent][K]).
  int r, c;
  if constexpr (TRANS_CONTIG_K) {
    r = f / kBK;
    c = f % kBK;
  } else {
    c = f / kTile;
    r = f % kTile;
  }
  *idx = r;
  *kk = c;
  const int gr = base + r, gk = k0 + c;
  if (gr >= extent || gk >= K) return T(0);
  return TRANS_CONTIG_K ? p[int64_t(gr) * ld + gk] : p[int64_t(gk) * ld + gr];
}

// A is op(A)[m][k]: stored [m][k] (contiguous in k) unless TA.
// B is op(B)[k][n]: stored [k][n] (contiguous in n) unless TB.
template <typename T, bool TA, bool TB, int PER>
struct TileLoader {
  T av[PER], bv[PER];
  int ai[PER], ak[PER], bi[PER], bk[PER];

  __device__ __forceinline__ void load(const TypedArgs& g, int m0, int n0, int k0) {
    const T* A = static_cast<const T*>(g.a);
    const T* B = static_cast<const T*>(g.b);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int f = threadIdx.x + j * kThreads;
      av[j] = load_elem<T, !TA>(A, g.lda, f, m0, k0, g.m, g.k, &ai[j], &ak[j]);
      bv[j] = load_elem<T, TB>(B, g.ldb, f, n0, k0, g.n, g.k, &bi[j], &bk[j]);
    }
  }
  // LDS layout: As[k][m], Bs[k][n] (pitch kTile + 1).
  __device__ __forceinline__ void store(T* As, T* Bs) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      As[ak[j] * (kTile + 1) + ai[j]] = av[j];
      Bs[bk[j] * (kTile + 1) + bi[j]] = bv[j];
    }
  }
};

constexpr int kPer = kTile * kBK / kThreads;  // 4 elements of A and of B per thread
constexpr int kLds = kBK * (kTile + 1);

// ------------------------------------------------------------------ float64


// float64, large products: 128 x 128 tiles of 4 waves, each wave 64 x 64 =
// 4 x 4 blocks of 16 x 16.  Per K step of 16 a workgroup moves 32 KiB from
// L2 into LDS for 64 MFMAs per wave, a quarter of the 64 x 64 kernel's
// traffic per flop, which leaves that kernel waiting on the L2 (61% MFMA busy
// at 4096^3).  K step, LDS tile, MFMA sequence and accumulator layout are the
// 64 x 64 kernel's, so both give the same bits; chosen once its tiles cover
// the CUs.  LDS rows are 129 doubles: an odd pitch spreads the k rows that a
// wave writes with one instruction over the banks (a pitch of 132 gave 4-way
// conflicts, a third of LDS-active cycles).
//
// Loads.  Each thread moves 4 pairs of adjacent doubles of each operand per K
// step with 16-byte loads.  A tile that lies wholly inside C, with both
// operands 16-byte aligned and of even leading dimension (TypedArgs::vec),
// runs every K step but the last in a loop of its own with unchecked loads:
// that loop is one basic block, so its loads, LDS reads, MFMAs and LDS stores
// can be interleaved.  The checked pair loads (edge tiles, the last K step)
// fill the same LDS tile, so every path gives the same bits.
constexpr int kBig = 128, kBigPitch = kBig + 1;

// One operand's share of a [TILE x 16] tile.  Pair q of thread tid is
// p = tid + 256 q.  KC (the stored matrix is contiguous along k): row
// r = p / 8 of the m (or n) extent and k offset c = 2 (p % 8); otherwise k
// row r = p / (TILE / 2) and m (or n) offset c = 2 (p % (TILE / 2)).  In LDS
// the tile is [k][m or n] with row pitch PITCH.
template <bool KC, int TILE = kBig, int PITCH = kBigPitch>
struct PairOperand {
  static constexpr int kPairs = TILE * kBK / 2 / kThreads;  // 4 (128-wide tiles), 2 (64)
  static constexpr int kRowPairs = KC ? kBK / 2 : TILE / 2;
  v2d v[kPairs];
  const double* at[kPairs];  // pair start at k0 = 0, for tiles inside the matrix

  __device__ __forceinline__ void init(const double* X, int ld, int base, int tid) {
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
      const int p = tid + kThreads * q, r = p / kRowPairs, c = 2 * (p % kRowPairs);
      at[q] = KC ? X + int64_t(base + r) * ld + c : X + int64_t(r) * ld + base + c;
    }
  }
  __device__ __forceinline__ void load_unchecked(int k0, int ld) {
#pragma unroll
    for (int q = 0; q < kPairs; ++q)
      v[q] = *reinterpret_cast<const v2d*>(KC ? at[q] + k0 : at[q] + int64_t(k0) * ld);
  }
  __device__ __forceinline__ void load_checked(const double* X, int ld, int base, int extent,
                                               int k0, int K, int tid) {
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
      const int p = tid + kThreads * q, r = p / kRowPairs, c = 2 * (p % kRowPairs);
      if constexpr (KC) {
        const int row = base + r, kk = k0 + c;
        const double* x = X + int64_t(row) * ld + kk;
        v[q].x = (row < extent && kk < K) ? x[0] : 0.0;
        v[q].y = (row < extent && kk + 1 < K) ? x[1] : 0.0;
      } else {
        const int kk = k0 + r, col = base + c;
        const double* x = X + int64_t(kk) * ld + col;
        v[q].x = (kk < K && col < extent) ? x[0] : 0.0;
        v[q].y = (kk < K && col + 1 < extent) ? x[1] : 0.0;
      }
    }
  }
  __device__ __forceinline__ void store(double* S, int tid) const {
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
      const int p = tid + kThreads * q, r = p / kRowPairs, c = 2 * (p % kRowPairs);
      if constexpr (KC) {
        S[c * PITCH + r] = v[q].x;
        S[(c + 1) * PITCH + r] = v[q].y;
      } else {
        S[r * PITCH + c] = v[q].x;
        S[r * PITCH + c + 1] = v[q].y;
      }
    }
  }
};

// Order of one unchecked K step, for the compiler's scheduler (masks: 0x8
// MFMA, 0x20 global load, 0x100 LDS read, 0x200 LDS write).  The first step's
// LDS reads, then the 8 loads of the next tile one per MFMA; each later
// step's 4 LDS reads are issued halfway through the previous step's 16 MFMAs;
// the 8 LDS stores of the next tile go one per MFMA among the last 8.
// Measured at 4096^3: 1.87 ms against 2.05 ms with LDS reads a whole step
// ahead and 2.12 ms for the compiler's own order.
__device__ __forceinline__ void f64_step_schedule() {
  __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
}

// float64 on 64 x 64 tiles of 4 waves, each wave 2 x 2 blocks of 16 x 16, for
// products whose 128 x 128 tiles do not cover the CUs.  Loads as in
// gemm_f64_big (pairs of the [64 x 16] panels, unchecked for aligned tiles
// inside C, checked otherwise, the same LDS tile either way); each unchecked
// K step puts the 4 loads of the next tile one per MFMA at its start and the
// LDS stores one per MFMA among its last MFMAs.  Measured against its
// element-wise checked loads: 1024^3 71-77 -> 60-64 us, 1536^3 206-214 ->
// 176-191 us (three orientations each).
template <bool TA, bool TB>
__global__ __launch_bounds__(kThreads) void gemm_f64_mfma(TypedArgs g) {
  __shared__ double smem[2][2][kLds];  // [buffer][A|B], each [k][m or n], pitch kTile + 1
  const int tiles_n = (g.n + kTile - 1) / kTile;
  const int m0 = int(blockIdx.x / tiles_n) * kTile, n0 = int(blockIdx.x % tiles_n) * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, lk = lane >> 4;
  const double* A = static_cast<const double*>(g.a);
  const double* B = static_cast<const double*>(g.b);
  PairOperand<!TA, kTile, kTile + 1> pa;
  PairOperand<TB, kTile, kTile + 1> pb;
  pa.init(A, g.lda, m0, tid);
  pb.init(B, g.ldb, n0, tid);
  const bool inside = g.vec && m0 + kTile <= g.m && n0 + kTile <= g.n && g.k >= kBK;
  auto load_checked = [&](int k0) {
    pa.load_checked(A, g.lda, m0, g.m, k0, g.k, tid);
    pb.load_checked(B, g.ldb, n0, g.n, k0, g.k, tid);
  };
  auto store = [&](int buf) {
    pa.store(smem[buf][0], tid);
    pb.store(smem[buf][1], tid);
  };

  v4d acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};
  auto compute = [&](int cur) {
    const double* As = smem[cur][0];
    const double* Bs = smem[cur][1];
#pragma unroll
    for (int s = 0; s < kBK / 4; ++s) {
      const int kk = 4 * s + lk;
      double af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = As[kk * (kTile + 1) + wm * 32 + i * 16 + li];
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = Bs[kk * (kTile + 1) + wn * 32 + j * 16 + li];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  const int k_tiles = (g.k + kBK - 1) / kBK;
  // Steps kt < unchecked_end load tile kt + 1, which lies wholly inside K.
  const int unchecked_end = inside ? g.k / kBK - 1 : 0;
  if (inside) {
    pa.load_unchecked(0, g.lda);
    pb.load_unchecked(0, g.ldb);
  } else {
    load_checked(0);
  }
  store(0);
  __syncthreads();
  int kt = 0;
  for (; kt < unchecked_end; ++kt) {
    const int cur = kt & 1;
    pa.load_unchecked((kt + 1) * kBK, g.lda);
    pb.load_unchecked((kt + 1) * kBK, g.ldb);
    compute(cur);
    store(cur ^ 1);
    // masks: 0x8 MFMA, 0x20 global load, 0x100 LDS read, 0x200 LDS write
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __syncthreads();
  }
  for (; kt < k_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_checked((kt + 1) * kBK);
    compute(cur);
    if (more) store(cur ^ 1);
    __syncthreads();
  }

  double* C = static_cast<double*>(g.c);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 32 + j * 16 + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 32 + i * 16 + 4 * r + lk;
        if (row < g.m && col < g.n) {
          double* p = C + int64_t(row) * g.ldc + col;
          *p = g.accumulate ? *p + acc[i][j][r] : acc[i][j][r];
        }
      }
    }
}

template <bool TA, bool TB>
__global__ __launch_bounds__(kThreads, 2) void gemm_f64_big(TypedArgs g) {
  __shared__ double As[2][kBK * kBigPitch], Bs[2][kBK * kBigPitch];  // [k][m], [k][n]
  const int tiles_n = (g.n + kBig - 1) / kBig;
  const int m0 = int(blockIdx.x / tiles_n) * kBig, n0 = int(blockIdx.x % tiles_n) * kBig;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, lk = lane >> 4;
  const double* A = static_cast<const double*>(g.a);
  const double* B = static_cast<const double*>(g.b);

  // A is op(A)[m][k], stored [m][k] (contiguous in k) unless TA; B is
  // op(B)[k][n], stored [k][n] unless TB (then [n][k], contiguous in k).
  PairOperand<!TA> pa;
  PairOperand<TB> pb;
  pa.init(A, g.lda, m0, tid);
  pb.init(B, g.ldb, n0, tid);
  const bool inside = g.vec && m0 + kBig <= g.m && n0 + kBig <= g.n && g.k >= kBK;
  auto load_checked = [&](int k0) {
    pa.load_checked(A, g.lda, m0, g.m, k0, g.k, tid);
    pb.load_checked(B, g.ldb, n0, g.n, k0, g.k, tid);
  };
  auto store = [&](int buf) {
    pa.store(As[buf], tid);
    pb.store(Bs[buf], tid);
  };

  v4d acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};
  auto compute = [&](int cur) {
    const double* as = As[cur];
    const double* bs = Bs[cur];
#pragma unroll
    for (int s = 0; s < kBK / 4; ++s) {
      const int kk = 4 * s + lk;
      double af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = as[kk * kBigPitch + wm * 64 + i * 16 + li];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = bs[kk * kBigPitch + wn * 64 + j * 16 + li];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  const int k_tiles = (g.k + kBK - 1) / kBK;
  // Steps kt < unchecked_end load tile kt + 1, which lies wholly inside K.
  const int unchecked_end = inside ? g.k / kBK - 1 : 0;
  if (inside) {
    pa.load_unchecked(0, g.lda);
    pb.load_unchecked(0, g.ldb);
  } else {
    load_checked(0);
  }
  store(0);
  __syncthreads();
  int kt = 0;
  for (; kt < unchecked_end; ++kt) {
    const int cur = kt & 1;
    pa.load_unchecked((kt + 1) * kBK, g.lda);
    pb.load_unchecked((kt + 1) * kBK, g.ldb);
    compute(cur);
    store(cur ^ 1);
    f64_step_schedule();
    __syncthreads();
  }
  for (; kt < k_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_checked((kt + 1) * kBK);
    compute(cur);
    if (more) store(cur ^ 1);
    __syncthreads();
  }

  double* C = static_cast<double*>(g.c);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn * 64 + j * 16 + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + 4 * r + lk;
        if (row < g.m && col < g.n) {
          double* p = C + int64_t(row) * g.ldc + col;
          *p = g.accumulate ? *p + acc[i][j][r] : acc[i][j][r];
        }
      }
    }
}

// ------------------------------------------------------------ bool / ints

// Accumulator of each output type: wrap-around unsigned arithmetic of the
// output's width (int16 accumulates in 32 bits and is truncated on store,
// which is the same residue), or OR of ANDs for bool.
template <typename T> struct IntAcc { using U = std::make_unsigned_t<T>; };
template <> struct IntAcc<int16_t> { using U = uint32_t; };
template <> struct IntAcc<bool> { using U = bool; };

template <typename T>
__device__ __forceinline__ typename IntAcc<T>::U mac(typename IntAcc<T>::U acc, T a, T b) {
  using U = typename IntAcc<T>::U;
  if constexpr (std::is_same_v<T, bool>) {
    return acc || (a && b);
  } else {
    return U(acc + U(U(a) * U(b)));
  }
}

template <typename T, bool TA, bool TB>
__global__ __launch_bounds__(kThreads) void gemm_int(TypedArgs g) {
  using U = typename IntAcc<T>::U;
  __shared__ T As[kLds], Bs[kLds];
  const int tiles_n = (g.n + kTile - 1) / kTile;
  const int m0 = int(blockIdx.x / tiles_n) * kTile, n0 = int(blockIdx.x % tiles_n) * kTile;
  const int tr = threadIdx.x / 16, tc = threadIdx.x % 16;  // rows tr + 16i, cols tc + 16j
  U acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = U(0);

  TileLoader<T, TA, TB, kPer> ld;
  for (int k0 = 0; k0 < g.k; k0 += kBK) {
    ld.load(g, m0, n0, k0);
    ld.store(As, Bs);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      T a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk * (kTile + 1) + tr + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk * (kTile + 1) + tc + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mac<T>(acc[i][j], a[i], b[j]);
    }
    __syncthreads();
  }

  T* C = static_cast<T*>(g.c);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = m0 + tr + 16 * i, col = n0 + tc + 16 * j;
      if (row >= g.m || col >= g.n) continue;
      T* p = C + int64_t(row) * g.ldc + col;
      if constexpr (std::is_same_v<T, bool>) {
        *p = g.accumulate ? (*p || acc[i][j]) : acc[i][j];
      } else {
        *p = g.accumulate ? T(U(U(*p) + acc[i][j])) : T(acc[i][j]);
      }
    }
}

template <typename T, bool TA, bool TB>
void launch_typed(Runtime* rt, const TypedArgs& g) {
  const int64_t tiles = int64_t((g.m + kTile - 1) / kTile) * ((g.n + kTile - 1) / kTile);
  const int64_t big_tiles = int64_t((g.m + kBig - 1) / kBig) * ((g.n + kBig - 1) / kBig);
  if constexpr (std::is_same_v<T, double>) {
    if (big_tiles >= rt->cu_count)
      hipLaunchKernelGGL((gemm_f64_big<TA, TB>), dim3(uint32_t(big_tiles)), dim3(kThreads), 0,
                         rt->stream, g);
    else
      hipLaunchKernelGGL((gemm_f64_mfma<TA, TB>), dim3(uint32_t(tiles)), dim3(kThreads), 0,
                         rt->stream, g);
  } else {
    hipLaunchKernelGGL((gemm_int<T, TA, TB>), dim3(uint32_t(tiles)), dim3(kThreads), 0,
                       rt->stream, g);
  }
}

template <typename T>
int dispatch_typed(Runtime* rt, bool ta, bool tb, const TypedArgs& g) {
  if (!ta && !tb) launch_typed<T, false, false>(rt, g);
  else if (!ta && tb) launch_typed<T, false, true>(rt, g);
  else if (ta && !tb) launch_typed<T, true, false>(rt, g);
  else launch_typed<T, true, true>(rt, g);
  LMP_LAUNCH_CHECK("gemm (typed)");
  return LMP_OK;
}

}  // namespace
}  // namespace lmp_hip

using namespace lmp_hip;

extern "C" int lmp_k_gemm(int dtype, int trans_a, int trans_b, size_t m, size_t n, size_t k,
                          const void* a, size_t lda, const void* b, size_t ldb, void* c,
                          size_t ldc, int accumulate) {
  if (dtype == LMP_FLOAT32)
    return lmp_k_gemm_f32(trans_a, trans_b, m, n, k, static_cast<const float*>(a), lda,
                          static_cast<const float*>(b), ldb, static_cast<float*>(c), ldc,
                          accumulate);
  if (dtype != LMP_FLOAT64 && dtype != LMP_INT64 && dtype != LMP_INT32 &&
      dtype != LMP_INT16 && dtype != LMP_BOOL)
    return fail(LMP_ERR_INVALID, "gemm: unknown dtype");
  if (m == 0 || n == 0) return LMP_OK;
  if (!c) return fail(LMP_ERR_INVALID, "gemm: null output");
  if (k == 0) {
    if (accumulate) return LMP_OK;
    if (ldc != n) return fail(LMP_ERR_UNSUPPORTED, "gemm: k == 0 with ldc != n");
    return lmp_k_fill(dtype, c, m * n, 0.0);
  }
  if (!a || !b) return fail(LMP_ERR_INVALID, "gemm: null input");
  const size_t lim = kGemmMaxExtent - 1;
  if (m > lim || n > lim || k > lim || lda > lim || ldb > lim || ldc > lim)
    return fail(LMP_ERR_UNSUPPORTED, "gemm: dimension of 2^31 - 4096 or more");
  if ((trans_a ? lda < m : lda < k) || (trans_b ? ldb < k : ldb < n) || ldc < n)
    return fail(LMP_ERR_INVALID, "gemm: leading dimension too small");
  const uint64_t tiles = uint64_t((m + kTile - 1) / kTile) * ((n + kTile - 1) / kTile);
  if (tiles > 0x7fffffffull) return fail(LMP_ERR_UNSUPPORTED, "gemm: grid too large");
  LMP_RUNTIME_OR_FAIL(rt);
  const bool vec = reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(b) % 16 == 0 && lda % 2 == 0 && ldb % 2 == 0;
  TypedArgs g{a, b, c, int(m), int(n), int(k), int(lda), int(ldb), int(ldc),
              accumulate ? 1 : 0, vec ? 1 : 0};
  const bool ta = trans_a != 0, tb = trans_b != 0;
  switch (dtype) {
    case LMP_FLOAT64: return dispatch_typed<double>(rt, ta, tb, g);
    case LMP_INT64: return dispatch_typed<int64_t>(rt, ta, tb, g);
    case LMP_INT32: return dispatch_typed<int32_t>(rt, ta, tb, g);
    case LMP_INT16: return dispatch_typed<int16_t>(rt, ta, tb, g);
    default: return dispatch_typed<bool>(rt, ta, tb, g);
  }
}
