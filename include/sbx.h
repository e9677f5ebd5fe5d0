/*
 * sbx.h -- C ABI of the MI355X (gfx950) GEMM hot path of SushiBLAS.
 *
 * This is the drop-in boundary.  In the reference, Level3::gemm
 * (src/ops/blas/level3/gemm.cpp:82-198) records a task whose body,
 * gemm_dispatch<T> (gemm.cpp:44-79), calls oneMKL on a sycl::queue.  Each
 * entry point below replaces one of those oneMKL calls one-for-one: the same
 * argument set as gemm_dispatch (gemm.cpp:45-51), with the sycl::queue
 * replaced by a hipStream_t and the dependency-event vector replaced by
 * stream order.
 *
 * Conventions
 *   - Plain pointers and sizes only; every buffer is caller-owned device
 *     memory (or pinned host memory mapped into the device address space).
 *     The library never frees or retains a caller pointer.
 *   - Launches are asynchronous on `stream` (NULL = the null stream of the
 *     current device; hipStreamPerThread is accepted).  The only allocation
 *     is the workspace for split-K GEMM/SYRK partials and chunked GEMV
 *     partials: cached per (device, stream), grown with hipMalloc (at least
 *     doubling) the first time a larger one is needed and reused after that;
 *     an outgrown buffer is kept, not freed, until the process ends.  Uses of
 *     a workspace are ordered by its stream.  Calls on hipStreamPerThread get
 *     no workspace and run unsplit.  If the allocation fails the call runs
 *     without splitting instead of failing.
 *   - Return value is a status code (sbx_status); nothing throws across the
 *     ABI.  The C++ layer turns codes into std::runtime_error, as the
 *     reference's SB_THROW_IF does (include/SushiBLAS/core/logger.hpp:316-323).
 *   - BLAS semantics: m == 0 || n == 0 is a no-op; alpha == 0 || k == 0 gives
 *     C = beta*C; beta == 0 means C is never read (NaN/Inf in C do not
 *     propagate).
 *   - layout 0 = row-major, 1 = column-major (Core::Layout,
 *     include/SushiBLAS/core/common.hpp:41-45).  transA/transB: 0 or 1.
 *   - Re-entrant: the only global state is the per-device CU count and the
 *     workspace cache, both behind mutexes; safe to call from any host thread
 *     (the reference runs the GEMM closure on a scheduler worker thread).
 *     Calls on one stream share its workspace and run in stream order; the
 *     two kernels of a split call are enqueued under that stream's lock, so
 *     concurrent host threads on one stream cannot interleave with them.
 */
#ifndef SBX_H
#define SBX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum sbx_status {
    SBX_OK = 0,
    SBX_INVALID_ARGUMENT = 1, /* bad layout/trans flag, negative size, ld too small, null ptr */
    SBX_UNSUPPORTED = 2,      /* dtype or shape this build cannot run                       */
    SBX_HIP_ERROR = 3         /* a HIP runtime call or kernel launch failed                */
} sbx_status;

typedef enum sbx_dtype { SBX_F32 = 0, SBX_F64 = 1 } sbx_dtype;

/* Replaces oneapi::mkl::blas::row_major::gemm<float> (gemm.cpp:63) and
 * column_major::gemm<float> (gemm.cpp:76), reached from the FLOAT32 case of
 * Level3::gemm (gemm.cpp:146-157). */
int sbx_sgemm(void* stream, int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              float alpha, const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
              float* C, int64_t ldc);

/* Replaces row_major::gemm<double> (gemm.cpp:63) / column_major::gemm<double>
 * (gemm.cpp:76), reached from the FLOAT64 case (gemm.cpp:158-169), where the
 * float alpha/beta are widened to double (gemm.cpp:161). */
int sbx_dgemm(void* stream, int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              double alpha, const double* A, int64_t lda, const double* B, int64_t ldb,
              double beta, double* C, int64_t ldc);

/* Replaces row_major::gemm_batch<float> (gemm.cpp:58) and
 * column_major::gemm_batch<float> (gemm.cpp:71): `batch` problems, problem b
 * using A + b*str_a, B + b*str_b, C + b*str_c (strides in elements, as
 * derived at gemm.cpp:103-105). */
int sbx_sgemm_strided_batched(void* stream, int layout, int transA, int transB, int64_t m,
                              int64_t n, int64_t k, float alpha, const float* A, int64_t lda,
                              int64_t str_a, const float* B, int64_t ldb, int64_t str_b,
                              float beta, float* C, int64_t ldc, int64_t str_c, int64_t batch);

/* Replaces row_major::gemm_batch<double> (gemm.cpp:58) / column_major::gemm_batch<double>
 * (gemm.cpp:71). */
int sbx_dgemm_strided_batched(void* stream, int layout, int transA, int transB, int64_t m,
                              int64_t n, int64_t k, double alpha, const double* A, int64_t lda,
                              int64_t str_a, const double* B, int64_t ldb, int64_t str_b,
                              double beta, double* C, int64_t ldc, int64_t str_c,
                              int64_t batch);

/* Algorithm override for tests and tuning (no counterpart in the reference,
 * where oneMKL chooses internally): SBX_ALGO_AUTO is what the four entry
 * points above use.  SBX_ALGO_MFMA: any MFMA kernel (model's choice);
 * SBX_ALGO_MFMA_TILE: the LDS-tiled MFMA kernels only; SBX_ALGO_MFMA_SMALL:
 * the one-launch small-problem kernel.  A forced choice the
 * problem cannot use returns SBX_UNSUPPORTED. */
typedef enum sbx_algo {
    SBX_ALGO_AUTO = 0,
    SBX_ALGO_GENERIC = 1,
    SBX_ALGO_MFMA = 2,
    SBX_ALGO_MFMA_TILE = 3,
    SBX_ALGO_MFMA_SMALL = 4
} sbx_algo;

/* dtype-generic form of the four entry points above; alpha/beta point to a
 * float (SBX_F32) or double (SBX_F64). */
int sbx_gemm_ex(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                int64_t str_a, const void* B, int64_t ldb, int64_t str_b, const void* beta,
                void* C, int64_t ldc, int64_t str_c, int64_t batch, int algo);

/* Bytes of the fixed per-device scratch that sbx_gemm_ex_noalloc uses. */
#define SBX_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* sbx_gemm_ex without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments and results as sbx_gemm_ex, except that split-K partials go to a
 * fixed array of SBX_NOALLOC_SCRATCH_BYTES in device memory (one per GPU,
 * held from the library's first use on that GPU until the process ends)
 * instead of the stream's workspace, and the tiling heuristics only consider
 * splits whose partials fit in it (a problem whose preferred split would not
 * fit runs with fewer k-parts or unsplit, so results may differ from
 * sbx_gemm_ex by rounding only; none is refused for its size).  It calls no
 * hipMalloc/hipFree.  Every call on one GPU shares that GPU's array.  A call
 * that splits holds a per-GPU host lock while it enqueues its two kernels
 * (the partial pass and the reduction), so concurrent host threads are
 * serialised at enqueue: on one stream, one call's kernels never interleave
 * with another's, whatever thread issued them.  Calls on different streams
 * of one GPU are not ordered by that lock: when their kernels run at the
 * same time they race on the array, and the caller must order them (one
 * stream, or events).  Every partial is written before it is read, so
 * nothing in the array needs clearing. */
int sbx_gemm_ex_noalloc(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                        int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                        int64_t str_a, const void* B, int64_t ldb, int64_t str_b,
                        const void* beta, void* C, int64_t ldc, int64_t str_c, int64_t batch,
                        int algo);

/* Epilogues that can be fused into the GEMM (no counterpart on the
 * reference's GEMM path, where they are separate tasks). */
typedef enum sbx_epilogue { SBX_EPILOGUE_NONE = 0, SBX_EPILOGUE_RELU = 1 } sbx_epilogue;

/* C = epilogue(alpha*op(A)*op(B) + beta*C), same arguments as sbx_gemm_ex.
 * SBX_EPILOGUE_RELU fuses the caller pattern of the reference's integration
 * tests -- Level3::gemm followed by NonLinearOps::relu on C
 * (tests/runtime/test_framework_sim.cpp:51-57,109-110; ReLU is
 * src/ops/math/nonlinear/relu.cpp:38-41: x > 0 ? x : 0) -- into one kernel,
 * saving the extra read and write of C. */
int sbx_gemm_fused(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                   int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                   int64_t str_a, const void* B, int64_t ldb, int64_t str_b, const void* beta,
                   void* C, int64_t ldc, int64_t str_c, int64_t batch, int epilogue);

/* Grouped GEMM: `count` problems C_i = epilogue(alpha*op(A_i)*op(B_i) +
 * beta*C_i) with one shape, one set of leading dimensions and scalars, and
 * operands anywhere in device memory: `table` is a DEVICE array of 3*count
 * pointers (A_0, B_0, C_0, A_1, B_1, C_1, ...), read by the kernel in stream
 * order.  aligned16 != 0 promises every C pointer is 16-byte aligned (enables
 * 16-byte C stores; operand loads are 16 bytes at any alignment).  One launch for all of them.  No single counterpart in the
 * reference: it is how the task graph issues a run of independent,
 * same-shaped Level3::gemm tasks (each one gemm.cpp:63 / :76 call in the
 * reference, run on worker threads) without one launch per task. */
int sbx_gemm_grouped(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                     int64_t n, int64_t k, const void* alpha, int64_t lda, int64_t ldb,
                     const void* beta, int64_t ldc, const void* const* table, int64_t count,
                     int aligned16, int epilogue);

/* x[i] = x[i] > 0 ? x[i] : 0 for n contiguous elements of dtype: the
 * stand-alone ReLU (replaces the body of NonLinearOps::relu,
 * src/ops/math/nonlinear/relu.cpp:38-41, for FLOAT32/FLOAT64). */
int sbx_relu(void* stream, int dtype, void* x, int64_t n);

/* GEMV, y = alpha*op(A)*x + beta*y with op(A) = A (m x n) or A^T: replaces
 * oneapi::mkl::blas::row_major::gemv (src/ops/blas/level2/gemv.cpp:55) and
 * column_major::gemv (gemv.cpp:60), reached from Level2::gemv (gemv.cpp:65-148)
 * for FLOAT32 / FLOAT64 (float alpha/beta widened, gemv.cpp:125).  x has
 * (transA ? m : n) elements x[i*incx], y has (transA ? n : m) elements
 * y[i*incy]; increments must be positive (the reference passes 1 or a rank-1
 * tensor's stride, utils.hpp:47-60).  Netlib quick returns: m == 0 or n == 0
 * leaves y untouched; alpha == 0 gives y = beta*y; beta == 0 never reads y. */
int sbx_sgemv(void* stream, int layout, int transA, int64_t m, int64_t n, float alpha,
              const float* A, int64_t lda, const float* x, int64_t incx, float beta, float* y,
              int64_t incy);
int sbx_dgemv(void* stream, int layout, int transA, int64_t m, int64_t n, double alpha,
              const double* A, int64_t lda, const double* x, int64_t incx, double beta,
              double* y, int64_t incy);

/* SYRK on one triangle of the n x n C: C = alpha*op(A)*op(A)^T + beta*C with
 * op(A) = A (n x k) when trans == 0 and A^T (A is k x n) when trans == 1;
 * upper != 0 updates the upper triangle, else the lower; the other triangle
 * is neither read nor written.  Replaces row_major::syrk / syrk_batch
 * (src/ops/blas/level3/syrk.cpp:65,60) and column_major::syrk / syrk_batch
 * (syrk.cpp:78,73), reached from Level3::syrk (syrk.cpp:84-194); batch b uses
 * A + b*str_a and C + b*str_c.  Quick returns as for GEMM: n == 0 is a
 * no-op, alpha == 0 or k == 0 gives C = beta*C on the triangle. */
int sbx_ssyrk(void* stream, int layout, int upper, int trans, int64_t n, int64_t k, float alpha,
              const float* A, int64_t lda, float beta, float* C, int64_t ldc);
int sbx_dsyrk(void* stream, int layout, int upper, int trans, int64_t n, int64_t k,
              double alpha, const double* A, int64_t lda, double beta, double* C, int64_t ldc);
int sbx_ssyrk_strided_batched(void* stream, int layout, int upper, int trans, int64_t n,
                              int64_t k, float alpha, const float* A, int64_t lda, int64_t str_a,
                              float beta, float* C, int64_t ldc, int64_t str_c, int64_t batch);
int sbx_dsyrk_strided_batched(void* stream, int layout, int upper, int trans, int64_t n,
                              int64_t k, double alpha, const double* A, int64_t lda,
                              int64_t str_a, double beta, double* C, int64_t ldc, int64_t str_c,
                              int64_t batch);

/* Name of the kernel the dispatcher would launch for this problem (tiling
 * heuristics introspection for benchmarks).  Pointers are assumed 16-byte
 * aligned.  Writes a NUL-terminated string of at most cap bytes. */
int sbx_gemm_select(int dtype, int layout, int transA, int transB, int64_t m, int64_t n,
                    int64_t k, int64_t lda, int64_t ldb, int64_t ldc, char* name, size_t cap);

/* The same for a strided batch of `batch` packed entries (stride = the stored
 * extent of each operand): a batch whose grid fills less than one round of
 * the device cuts K too, so its pick can differ from a single problem's.
 * No counterpart in the reference (introspection, as above). */
int sbx_gemm_select_batched(int dtype, int layout, int transA, int transB, int64_t m, int64_t n,
                            int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch,
                            char* name, size_t cap);

/* The plans the tiling heuristics weigh for this (packed, as above) problem:
 * one line "<plan name> <predicted microseconds>\n" per candidate kernel and
 * k-split, in the names sbx_gemm_select reports (NUL-terminated, at most cap
 * bytes; SBX_INVALID_ARGUMENT if they do not fit).  No counterpart in the
 * reference: it serves measurements of the heuristics against every
 * candidate (regret), with sbx_gemm_ex_plan. */
int sbx_gemm_plans(int dtype, int layout, int transA, int transB, int64_t m, int64_t n,
                   int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch, char* out,
                   size_t cap);

/* sbx_gemm_ex (algo = AUTO) with the named plan -- a name from sbx_gemm_plans
 * or sbx_gemm_select -- instead of the heuristics' pick.  Same results as any
 * plan within the tolerance.  SBX_INVALID_ARGUMENT for a name that is no
 * plan, SBX_UNSUPPORTED for a plan the problem cannot use (another element
 * type, offsets beyond the kernel's range, more k-ranges than its tail
 * allows).  No counterpart in the reference (measurement hook, as above). */
int sbx_gemm_ex_plan(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                     int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                     int64_t str_a, const void* B, int64_t ldb, int64_t str_b, const void* beta,
                     void* C, int64_t ldc, int64_t str_c, int64_t batch, const char* plan);

/* The same for sbx_{s,d}syrk[_strided_batched] (single problem): the kernel
 * and split that would compute the triangle. */
int sbx_syrk_select(int dtype, int layout, int upper, int trans, int64_t n, int64_t k,
                    int64_t lda, int64_t ldc, char* name, size_t cap);

/* sbx_gemm_plans for a single SYRK problem: the plans (square tile configs
 * over the triangle, unsplit and split) the heuristics weigh.  No counterpart
 * in the reference (measurement hook, as above). */
int sbx_syrk_plans(int dtype, int layout, int upper, int trans, int64_t n, int64_t k,
                   int64_t lda, int64_t ldc, char* out, size_t cap);

/* sbx_{s,d}syrk_strided_batched with the named plan (a name from
 * sbx_syrk_plans or sbx_syrk_select) instead of the heuristics' pick; status
 * as sbx_gemm_ex_plan (a config that is not a triangle's is
 * SBX_UNSUPPORTED).  alpha and beta point to the element type's scalar.  No
 * counterpart in the reference (measurement hook, as above). */
int sbx_syrk_ex_plan(void* stream, int dtype, int layout, int upper, int trans, int64_t n,
                     int64_t k, const void* alpha, const void* A, int64_t lda, int64_t str_a,
                     const void* beta, void* C, int64_t ldc, int64_t str_c, int64_t batch,
                     const char* plan);

/* Human-readable text for a status code (static storage). */
const char* sbx_status_string(int status);

/* Synthetic-input generators (Philox4x32-10, counter-based), writing n
 * elements of dtype into device memory on `stream`.  They stand in for the
 * reference's RandomOps::uniform / normal (src/ops/math/random/uniform.cpp:40-62)
 * only as a source of benchmark inputs; the stream layout is this library's
 * own: key = seed, counter = (element block, stream_id, 0).
 * uniform: [-1, 1).  normal: N(0, 1) * scale. */
int sbx_fill_uniform(void* stream, int dtype, void* out, int64_t n, uint64_t seed,
                     uint32_t stream_id);
int sbx_fill_normal(void* stream, int dtype, void* out, int64_t n, uint64_t seed,
                    uint32_t stream_id, double scale);

/* Library version string. */
const char* sbx_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SBX_H */
