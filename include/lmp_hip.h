/*
 * lmp_hip.h — C ABI of the MI355X (gfx950) device backend for Lamp3.
 *
 * This is the drop-in boundary.  Lamp3 reaches its GPU device through
 * per-device function-pointer tables (DispatchStub,
 * csrc/include/lamp3/tensor/dispatch_stub.hpp:21-64) and one lazy-backend slot
 * (csrc/include/lamp3/tensor/lazy/lazy_backend.hpp:15-35).  The CUDA backend
 * fills those slots with `*_cuda` functions; this library exports plain C
 * entry points that a `*_hip` adapter registered in the same slots calls
 * instead.  Each declaration below names the reference function it replaces.
 *
 * Conventions
 *  - Every entry point returns an lmp_status; LMP_OK (0) is success.  On
 *    failure lmp_rt_last_error() returns a thread-local message.
 *  - Pointers passed as "device" pointers must come from lmp_rt_malloc (or any
 *    other HIP device allocation on the current device).
 *  - All work is issued in order on one HIP stream owned by the library
 *    (lmp_rt_stream()).  Entry points that launch kernels return without
 *    synchronising; copies to host memory synchronise before returning.
 *  - dtype codes equal lmp::tensor::DataType (data_type.hpp:25-32).
 *  - Element strides are in elements, not bytes.  A stride of 0 marks a
 *    broadcast dimension (cpu/offset_util.cpp:7-28 pads size-1 dims with 0).
 */
#ifndef LMP_HIP_H_
#define LMP_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LMP_HIP_ABI_VERSION 9
#define LMP_MAX_DIMS 16 /* align_utils.hpp:7 */
/* Size of the fixed per-device workspace of lmp_k_gemm_f32_noalloc. */
#define LMP_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

typedef enum {
  LMP_OK = 0,
  LMP_ERR_INVALID = 1,     /* bad argument: shape, dtype, null pointer */
  LMP_ERR_RUNTIME = 2,     /* HIP runtime call failed */
  LMP_ERR_OOM = 3,         /* device allocation failed after cache release */
  LMP_ERR_UNSUPPORTED = 4, /* valid request this backend does not implement */
  LMP_ERR_JIT = 5          /* hipRTC compile or module load failed */
} lmp_status;

typedef enum { /* data_type.hpp:25-32 */
  LMP_BOOL = 0,
  LMP_INT16 = 1,
  LMP_INT32 = 2,
  LMP_INT64 = 3,
  LMP_FLOAT32 = 4,
  LMP_FLOAT64 = 5
} lmp_dtype;

/* Binary elementwise ops: native/expand_ops.hpp:11-33 and the two backward
 * functors of native/unary_ops.hpp:11-34 (functors: cpu/kernels.hpp:22-154). */
typedef enum {
  LMP_BIN_ADD = 0,
  LMP_BIN_SUB = 1,
  LMP_BIN_MUL = 2,
  LMP_BIN_DIV = 3,
  LMP_BIN_POW = 4,
  LMP_BIN_EQ = 5,
  LMP_BIN_NE = 6,
  LMP_BIN_GE = 7,
  LMP_BIN_LE = 8,
  LMP_BIN_GT = 9,
  LMP_BIN_LT = 10,
  LMP_BIN_ABS_BACKWARD = 11,   /* (input, grad) */
  LMP_BIN_CLAMP_BACKWARD = 12, /* (input, grad), bounds in p0/p1 */
  LMP_BIN_COUNT = 13
} lmp_binary_op;

/* Unary elementwise ops: native/unary_ops.hpp:11-34. */
typedef enum {
  LMP_UN_NEG = 0,
  LMP_UN_EXP = 1,
  LMP_UN_LOG = 2,
  LMP_UN_SQRT = 3,
  LMP_UN_ABS = 4,
  LMP_UN_SIN = 5,
  LMP_UN_COS = 6,
  LMP_UN_TAN = 7,
  LMP_UN_CLAMP = 8, /* bounds in p0/p1; ReLU is clamp(x, 0, DBL_MAX) */
  LMP_UN_COUNT = 9
} lmp_unary_op;

/* Reductions: native/reduct_ops.hpp:11-19, identities cpu/kernels.hpp:155-174 */
typedef enum {
  LMP_RED_SUM = 0,
  LMP_RED_MAX = 1,
  LMP_RED_MIN = 2,
  LMP_RED_PROD = 3,
  LMP_RED_COUNT = 4
} lmp_reduce_op;

/* Broadcast descriptor, passed by value into kernels (no per-op metadata
 * copies to the device, unlike offset_util.cu:20-29).  The output is the
 * contiguous tensor of `shape`; stride_a/stride_b are each input's element
 * strides aligned to the output dims, 0 where that input broadcasts. */
typedef struct {
  int32_t ndim;
  int64_t shape[LMP_MAX_DIMS];
  int64_t stride_a[LMP_MAX_DIMS];
  int64_t stride_b[LMP_MAX_DIMS];
} lmp_bcast;

typedef struct {
  int32_t device;
  int32_t cu_count;
  int32_t simd_per_cu;
  int32_t wave_size;
  int64_t lds_bytes_per_cu;
  int64_t total_mem_bytes;
  int32_t clock_khz;
  int32_t mem_clock_khz;
  int32_t mem_bus_width;
  char arch[64]; /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  char name[128];
} lmp_rt_info;

typedef struct {
  uint64_t reserved_bytes;  /* bytes held in segments from hipMalloc */
  uint64_t allocated_bytes; /* bytes handed out to callers */
  uint64_t segments;
  uint64_t allocs;          /* lifetime allocation count */
  uint64_t device_mallocs;  /* lifetime hipMalloc count */
} lmp_rt_pool_stats;

/* ---------------------------------------------------------------- runtime */

/* Select the device and create the library stream.  Idempotent.  Replaces the
 * implicit CUDA runtime initialisation of allocator.cu:82-90. */
int lmp_rt_init(int device);
int lmp_rt_device_count(int* count);
int lmp_rt_device_info(lmp_rt_info* info);
/* Thread-local message for the last failed call on this thread. */
const char* lmp_rt_last_error(void);
int lmp_rt_abi_version(void);

/* Pooled device allocation (best-fit arena, 256 B alignment, coalescing,
 * cache release and one retry on OOM).  Replaces empty_cuda (memory.cu:56-65)
 * -> CudaAllocator::allocate/deallocate (allocator.cu:48-80, BlockArena
 * allocator_core.hpp:33-207).  A zero-byte request returns NULL. */
int lmp_rt_malloc(void** ptr, size_t bytes);
int lmp_rt_free(void* ptr);
/* Return fully free segments to the HIP runtime (allocator.cu:117-125). */
int lmp_rt_empty_cache(void);
int lmp_rt_pool_stats_get(lmp_rt_pool_stats* stats);
/* Number of kernels this process has launched through the library: every
 * kernel of every entry point, hipRTC kernels included; a launch recorded into
 * a graph counts once, its replays do not.  No counterpart in the reference;
 * it lets a caller count the kernels of a step (measurement only). */
int lmp_rt_kernel_launch_count(uint64_t* count);

/* Copies on the library stream.  h2d/d2h synchronise before returning so the
 * host buffer may be reused or read; from 4 MiB up they run through pinned
 * staging buffers, host threads and the DMA engine overlapped chunk by chunk.
 * Replace the memcpy halves of copy_cuda / vecCopyHostToDevice
 * (memory.cu:103-174). */
int lmp_rt_memcpy_h2d(void* dst, const void* src, size_t bytes);
int lmp_rt_memcpy_d2h(void* dst, const void* src, size_t bytes);
int lmp_rt_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Wait for all work on the library stream (bindings/cuda.hpp:11-17). */
int lmp_rt_synchronize(void);
/* The hipStream_t every entry point launches on. */
void* lmp_rt_stream(void);

/* Timing events recorded on the library stream. */
int lmp_rt_event_create(void** event);
int lmp_rt_event_record(void* event);
int lmp_rt_event_elapsed_ms(void* start, void* stop, float* ms);
int lmp_rt_event_destroy(void* event);

/* HIP graphs: record the library stream's work once, replay it with one
 * launch.  No counterpart in the reference, which launches every kernel from
 * the host each step; here a whole training step (forward, backward, update)
 * can become one hipGraphLaunch.
 *   lmp_rt_graph_begin   start capturing the library stream.  Until end or
 *                        abort, kernel entry points record instead of run,
 *                        and lmp_rt_malloc serves the graph's private pool:
 *                        those blocks are never handed to eager allocations,
 *                        so replays cannot overwrite other tensors.
 *                        h2d/d2h copies, synchronize and event timing fail
 *                        with LMP_ERR_INVALID during a capture.
 *   lmp_rt_graph_end     close the capture and instantiate it (*graph).
 *   lmp_rt_graph_abort   close and discard an open capture (error paths).
 *   lmp_rt_graph_launch  enqueue one replay on the library stream.
 *   lmp_rt_graph_destroy free the graph; its pool's memory returns to HIP once
 *                        every block allocated in it has been freed.
 * Buffers allocated before the capture and read by it must outlive the graph.
 * One capture at a time, from one host thread. */
int lmp_rt_graph_begin(void);
int lmp_rt_graph_end(void** graph);
int lmp_rt_graph_abort(void);
int lmp_rt_graph_launch(void* graph);
int lmp_rt_graph_destroy(void* graph);

/* ------------------------------------------------------ elementwise kernels */

/* out[i] = op(a[ia(i)], b[ib(i)]) over the contiguous output of desc->shape.
 * All three buffers are of `dtype` (mixed-dtype callers cast first, which is
 * the cast-then-operate order of cpu/ptr_pack.hpp:9-35).  p0/p1 carry the
 * clamp bounds of LMP_BIN_CLAMP_BACKWARD.  Replaces the eleven binary
 * `*_cuda` entries (kernels.cu:13-29, registered kernels.cu:124-134) with
 * their kernels binary.cu:15-96 and expand.cu:14-59, plus abs_backward_cuda
 * and clamp_backward_cuda (kernels.cu:58-64, registered :145-148). */
int lmp_k_binary(int op, int dtype, void* out, const void* a, const void* b,
                 const lmp_bcast* desc, double p0, double p1);

/* out[i] = op(in[i]) for i < n.  Replaces the unary `*_cuda` entries and
 * clamp_cuda (kernels.cu:31-56, registered :136-144; kernels unary.cu). */
int lmp_k_unary(int op, int dtype, void* out, const void* in, size_t n,
                double p0, double p1);

/* out[i] = (dtype)value.  Replaces fill_cuda (memory.cu:67-73,191-204). */
int lmp_k_fill(int dtype, void* out, size_t n, double value);

/* dst[i] = (dst_dtype)src[i].  The device-side conversion of copy_cuda /
 * cudaVecCopy (memory.cu:176-189). */
int lmp_k_cast(int src_dtype, int dst_dtype, void* dst, const void* src,
               size_t n);

/* dst[i] += src[i].  Replaces add_inplace_cuda (memory.cu:22-54,75-83). */
int lmp_k_add_inplace(int dtype, void* dst, const void* src, size_t n);

/* ------------------------------------------------------------- reductions */

/* Keep-dims reduction of a contiguous tensor viewed as [outer, len, inner]
 * along the middle axis; out is [outer, inner].  Replaces sum/max/min/prod
 * _cuda (kernels.cu:112-122, registered :153-156) and the dispatcher
 * reduct.cu:213-260 with its kernels reduct.cu:15-150. */
int lmp_k_reduce(int op, int dtype, void* out, const void* in, size_t outer,
                 size_t len, size_t inner);

/* ----------------------------------------------------------------- matrix */

/* C[m,n] (+)= op(A)[m,k] * op(B)[k,n], row-major, fp32, fp32 MFMA
 * accumulation.  trans_a != 0 means A is stored [k,m] (lda >= m); trans_b != 0
 * means B is stored [n,k] (ldb >= k).  accumulate != 0 adds into C.
 * Replaces matmul_cuda -> cudaMatMul (kernels.cu:83-110, matrix.cu:21-199);
 * the transposed forms replace the transpose-then-matmul pairs of
 * MatrixMultiplicationBackward (functions/matrix_ops.cpp:8-24). */
int lmp_k_gemm_f32(int trans_a, int trans_b, size_t m, size_t n, size_t k,
                   const float* a, size_t lda, const float* b, size_t ldb,
                   float* c, size_t ldc, int accumulate);

/* lmp_k_gemm_f32 without allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Like every
 * kernel entry point it launches on the library stream (lmp_rt_stream()): a
 * capture records it when that stream is captured, by lmp_rt_graph_begin or
 * by a caller that makes the library stream wait on an event recorded in its
 * own capturing stream and joins back the same way.  Same arguments, kernels and results (bit for bit) as
 * lmp_k_gemm_f32; the split-K partials of products that split K go to a
 * fixed workspace of LMP_NOALLOC_SCRATCH_BYTES (a device array, one copy per
 * device, reserved when the library's code object loads there and held until
 * the process ends) instead of the pool.  A product whose partials would not
 * fit fails with LMP_ERR_UNSUPPORTED (lmp_k_gemm_f32 serves it); config 4's
 * largest split (512 x 4096, K split four ways) uses exactly 32 MiB.  Calls
 * allocate nothing and free nothing, and need nothing cleared between them
 * (every partial is written before it is read).  All calls on one GPU share
 * its workspace: calls whose kernels overlap on that GPU (graphs holding
 * them replayed concurrently on different streams) race.  The first call of
 * any entry point before lmp_rt_init performs the library's set-up. */
int lmp_k_gemm_f32_noalloc(int trans_a, int trans_b, size_t m, size_t n, size_t k,
                           const float* a, size_t lda, const float* b, size_t ldb,
                           float* c, size_t ldc, int accumulate);

/* C = op(A) * op(B) + bias, bias a row vector of n values added to every row
 * of the finished fp32 product (after any split-K fold): one pass instead of
 * the reference's matmul followed by a broadcast add (LinearImpl::forward,
 * layers/linear.cpp:21-26; linear.py:31-34).  Same rounding as the two-step
 * form: the product is complete before the bias is added, and it is the
 * product lmp_k_gemm_f32 computes (the same kernel whatever the bias; a bias
 * that is not 16-byte aligned is first copied to one that is), so the result
 * equals lmp_k_gemm_f32 then the add bit for bit. */
int lmp_k_linear_f32(int trans_a, int trans_b, size_t m, size_t n, size_t k,
                     const float* a, size_t lda, const float* b, size_t ldb,
                     const float* bias, float* c, size_t ldc);

/* C (+)= op(A) * op(B) and colsum[j] (+)= sum over k of op(B)[k][j]: a
 * Linear's weight gradient X^T dY and bias gradient (the dim-0 sum of dY)
 * together.  LinearBackward in the reference computes them apart: the bias
 * through AddBackward's grad-of-broadcast reduction (grad_utils.cpp:10-36)
 * and the weight through transpose + matmul (functions/matrix_ops.cpp:15-20).
 * The column sums ride in the GEMM's own launch on the tiny kernel (K <= 512,
 * at most 2^21 multiply-adds), on the LDS tiles when B is untransposed and K
 * is not split, and on the short-K kernel (A transposed, K <= 32); otherwise
 * a second launch forms them after the GEMM (the dim-0 reduction for a
 * contiguous B, a strided column sum for any ldb).  Anything the second launch
 * needs is reserved before the first, so an error return leaves C and colsum
 * unchanged.  accumulate / colsum_accumulate add into C / colsum instead of
 * writing. */
int lmp_k_gemm_colsum_f32(int trans_a, int trans_b, size_t m, size_t n, size_t k,
                          const float* a, size_t lda, const float* b, size_t ldb,
                          float* c, size_t ldc, int accumulate, float* colsum,
                          int colsum_accumulate);

/* lmp_k_gemm_colsum_f32 (B untransposed) with ReLU's backward applied to B
 * first: C (+)= op(A) * B' and colsum (+)= the column sums of B', where
 * B'[k][j] = B[k][j] if 0 < mask[k][j] < +inf, else +0.0 -- ClampBackward's
 * strict bounds for clamp(t, 0, DBL_MAX) (functions/unary_ops.cpp:27,
 * cpu/kernels.hpp:143-152), `mask` the ReLU output stored like B (ldb).  A
 * Linear -> ReLU pair's weight and bias gradients when its input needs no
 * gradient, without materialising the masked gradient: the reference runs
 * ReLU's backward, a transpose, a matmul and a reduction.  Small products
 * (K <= 512, at most 2^21 multiply-adds) mask B as it is loaded, in one
 * launch; larger ones mask into a scratch buffer, then take the column-sum
 * GEMM.  Same bits as the clamp-backward kernel followed by
 * lmp_k_gemm_colsum_f32. */
int lmp_k_gemm_colsum_masked_f32(int trans_a, size_t m, size_t n, size_t k,
                                 const float* a, size_t lda, const float* b,
                                 const float* mask, size_t ldb, float* c, size_t ldc,
                                 int accumulate, float* colsum, int colsum_accumulate);

/* The three gradients of a Linear y = x * w + b (x [batch, in] with row
 * stride ldx, w [in, out] with ldw) from its output gradient g [batch, out]
 * (ldg): dx (+)= g * w^T [batch, in] (lddx), dw (+)= x^T * g [in, out] (lddw)
 * and db (+)= the column sums of g [out]; each *_accumulate adds instead of
 * writing.  The reference forms them by MatrixMultiplicationBackward and the
 * broadcast add's sum (functions/matrix_ops.cpp:8-35, autograd/utils/
 * grad_utils.cpp:10-36): two transposes, two matmuls and a reduction.  When
 * both products fit the tiny GEMM's 16 x 16 blocks (K <= 512, at most 2^21
 * multiply-adds, blocks of 32 x 32 short of a quarter of the CUs) they run as
 * one launch; otherwise lmp_k_gemm_colsum_f32 (dw, db) then lmp_k_gemm_f32
 * (dx).  Either way the same bits as those two calls.  Argument errors are
 * returned before anything is written; after the first of the two calls only
 * running out of device memory can fail, which leaves dx unwritten. */
int lmp_k_linear_backward_f32(size_t batch, size_t in, size_t out, const float* x, size_t ldx,
                              const float* w, size_t ldw, const float* g, size_t ldg,
                              float* dx, size_t lddx, int dx_accumulate, float* dw,
                              size_t lddw, int dw_accumulate, float* db, int db_accumulate);

/* C = relu(op(A) * op(B) + bias): lmp_k_linear_f32 with ReLU applied in the
 * same epilogue, as the clamp functor computes clamp(t, 0, DBL_MAX) in float32
 * (t < 0 ? 0 : t; NaN and -0.0 pass through).  Replaces a Sequential's Linear
 * followed by ReLU (layers/linear.cpp:21-26 then layers/activation.cpp:14),
 * which the reference runs as matmul, broadcast add and clamp. */
int lmp_k_linear_relu_f32(int trans_a, int trans_b, size_t m, size_t n, size_t k,
                          const float* a, size_t lda, const float* b, size_t ldb,
                          const float* bias, float* c, size_t ldc);

/* The same product for any dtype, operands and C all of `dtype`
 * (LMP_FLOAT32 is lmp_k_gemm_f32).  float64 accumulates on the f64 matrix
 * cores; bool / int16 / int32 / int64 follow cpu/matrix.cpp:8-18 exactly:
 * the sum starts at 0 in the output type, so integers wrap modulo 2^bits and
 * bool is an OR of ANDs.  Replaces the remaining cudaMatMul instantiations
 * (matrix.cu:208-216) behind matmul_cuda (kernels.cu:83-110), whose callers
 * cast mixed operands to the promoted type first (cpu/matrix.cpp:8-18 casts
 * each operand to the output type). */
int lmp_k_gemm(int dtype, int trans_a, int trans_b, size_t m, size_t n, size_t k,
               const void* a, size_t lda, const void* b, size_t ldb, void* c,
               size_t ldc, int accumulate);

/* out[n,m] = in[m,n].  Replaces transpose_cuda / cudaTransposeKernel
 * (kernels.cu:66-81, matrix.cu:165-206). */
int lmp_k_transpose(int dtype, void* out, const void* in, size_t m, size_t n);

/* ------------------------------------------------------------- fusion JIT */

/* hipRTC module cache keyed by a caller-computed 64-bit graph hash.
 * lmp_jit_lookup returns LMP_OK with *handle set on a hit and LMP_ERR_INVALID
 * with *handle = NULL on a miss; lmp_jit_compile compiles `source` for the
 * current device's gfx target with -O3 -ffp-contract=off, loads it, resolves
 * `kernel_name` and caches it under `key`.  Replaces KernelCache /
 * compile_and_load (nvrtc_backend.cpp:54-128). */
int lmp_jit_lookup(uint64_t key, void** handle);
int lmp_jit_compile(uint64_t key, const char* source, const char* kernel_name,
                    void** handle);
/* Launch a cached kernel on the library stream with a 1-D grid; `args` holds
 * pointers to each kernel argument, as hipModuleLaunchKernel expects.  No
 * synchronisation (the reference synchronises every launch,
 * nvrtc_backend.cpp:135-141). */
int lmp_jit_launch(void* handle, uint32_t grid, uint32_t block, void** args);
/* Number of modules compiled by this process with hipRTC. */
int lmp_jit_compiled_count(uint64_t* count);
/* Number of modules this process loaded from the on-disk code-object cache
 * instead of compiling ($LMP_HIP_JIT_CACHE, default
 * ~/.cache/rushlite_amd/hiprtc; an empty value disables it).  No counterpart
 * in the reference, which compiles every graph again in each process
 * (nvrtc_backend.cpp:54-128). */
int lmp_jit_disk_loaded_count(uint64_t* count);

#ifdef __cplusplus
}
#endif

#endif /* LMP_HIP_H_ */
