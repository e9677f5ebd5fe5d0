/*
 * sbo.h -- CPU oracle for the SushiBLAS GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (sushiblas_amd/, include/)
 * includes, links or calls this.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker (or as the
 * timed CPU baseline), never as the thing that is measured or shipped.
 *
 * What it restates (all citations are into the read-only reference tree):
 *   - sbo_sgemm / sbo_dgemm and the strided-batched variants restate the
 *     arithmetic the reference delegates to oneMKL from gemm_dispatch<T>
 *     (src/ops/blas/level3/gemm.cpp:44-79): C = alpha*op(A)*op(B) + beta*C in
 *     row- or column-major storage, batch strides str_a/str_b/str_c
 *     (gemm.cpp:103-105), with the netlib/oneMKL quick-return rules
 *     (m==0||n==0: no-op; alpha==0||k==0: C = beta*C; beta==0: C not read).
 *     The oneMKL library itself (unpinned version, linked via -qmkl at
 *     src/CMakeLists.txt:139-143) is absent here, so the summation order is
 *     this file's own; parity is tolerance-based (normwise relative error).
 *   - sbo_gemm_naive_ld is an independent plain triple loop in long double
 *     over the same element accessors, used to check the blocked routine.
 *   - sbo_sgemv / sbo_dgemv restate Level2::gemv's oneMKL call
 *     (src/ops/blas/level2/gemv.cpp:44-61) and sbo_{s,d}syrk_strided_batched
 *     Level3::syrk's (src/ops/blas/level3/syrk.cpp:44-77): one double dot
 *     product per output element, netlib quick returns, SYRK touching only
 *     the requested triangle.
 *   - sbo_philox4x32_10 is the counter-based generator family the reference
 *     uses for its random ops (src/ops/math/random/uniform.cpp:47, oneMKL
 *     philox4x32x10); the algorithm is Salmon et al., "Parallel random
 *     numbers: as easy as 1, 2, 3" (SC'11).  The reference's own stream
 *     layout (skip_ahead(offset*size)) is NOT reproduced: inputs here come
 *     from this build's own counter mapping, identical on host and device.
 *
 * Pinning (what checks this file): the known answers of
 * tests/blas/level3/test_gemm.cpp:39-88, test_syrk.cpp and
 * tests/blas/level2/test_gemv.cpp, closed forms from
 * tests/runtime/test_framework_sim.cpp, brute force against
 * sbo_gemm_naive_ld, an independent host BLAS (numpy/OpenBLAS and
 * torch/MKL), transpose/column-major invariants, and the published
 * Random123 known-answer vectors for Philox4x32-10.  See tests/test_oracle.py.
 */
#ifndef SBO_H
#define SBO_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* acc_mode: 0 = accumulate in the storage type (what a vendor sgemm does),
 *           1 = accumulate in double (the "truth" used by parity tests).
 * For dgemm both modes accumulate in double.
 * layout:   0 = row-major, 1 = column-major (gemm.cpp:53-78). */
int sbo_sgemm(int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
              float beta, float* C, int64_t ldc, int acc_mode);
int sbo_dgemm(int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              double alpha, const double* A, int64_t lda, const double* B, int64_t ldb,
              double beta, double* C, int64_t ldc, int acc_mode);
int sbo_sgemm_strided_batched(int layout, int transA, int transB, int64_t m, int64_t n,
                              int64_t k, float alpha, const float* A, int64_t lda,
                              int64_t str_a, const float* B, int64_t ldb, int64_t str_b,
                              float beta, float* C, int64_t ldc, int64_t str_c,
                              int64_t batch, int acc_mode);
int sbo_dgemm_strided_batched(int layout, int transA, int transB, int64_t m, int64_t n,
                              int64_t k, double alpha, const double* A, int64_t lda,
                              int64_t str_a, const double* B, int64_t ldb, int64_t str_b,
                              double beta, double* C, int64_t ldc, int64_t str_c,
                              int64_t batch, int acc_mode);

/* Plain triple loop in long double (elem = 4: float, 8: double). */
int sbo_gemm_naive_ld(int elem, int layout, int transA, int transB, int64_t m, int64_t n,
                      int64_t k, double alpha, const void* A, int64_t lda, const void* B,
                      int64_t ldb, double beta, void* C, int64_t ldc);

/* ||X - Y||_F / ||Y||_F over an rows x cols row-major window (ld in elements). */
double sbo_rel_fro_err_f32(int64_t rows, int64_t cols, const float* X, int64_t ldx,
                           const float* Y, int64_t ldy);
double sbo_rel_fro_err_f64(int64_t rows, int64_t cols, const double* X, int64_t ldx,
                           const double* Y, int64_t ldy);

/* ReLU in place over n elements, as the reference defines it
 * (src/ops/math/nonlinear/relu.cpp:38-41): x > 0 ? x : 0, so NaN and -0
 * become +0. */
void sbo_relu_f32(float* x, int64_t n);
void sbo_relu_f64(double* x, int64_t n);

/* GEMV (src/ops/blas/level2/gemv.cpp:44-61, oneMKL gemv): y = alpha*op(A)*x
 * + beta*y, A m x n in `layout`, op(A) = A^T when trans; positive
 * increments.  Dot products in double, one rounding.  Netlib quick returns.
 * Returns 0, or 1 for invalid arguments. */
int sbo_sgemv(int layout, int trans, int64_t m, int64_t n, float alpha, const float* A,
              int64_t lda, const float* x, int64_t incx, float beta, float* y, int64_t incy);
int sbo_dgemv(int layout, int trans, int64_t m, int64_t n, double alpha, const double* A,
              int64_t lda, const double* x, int64_t incx, double beta, double* y, int64_t incy);

/* SYRK (src/ops/blas/level3/syrk.cpp:44-77, oneMKL syrk / syrk_batch): the
 * `upper` (j >= i) or lower (j <= i) triangle of the n x n C becomes
 * alpha*op(A)*op(A)^T + beta*C, op(A) = A (n x k) or A^T (A k x n); the
 * other triangle is untouched.  Sums in double, one rounding. */
int sbo_ssyrk_strided_batched(int layout, int upper, int trans, int64_t n, int64_t k,
                              float alpha, const float* A, int64_t lda, int64_t str_a,
                              float beta, float* C, int64_t ldc, int64_t str_c, int64_t batch);
int sbo_dsyrk_strided_batched(int layout, int upper, int trans, int64_t n, int64_t k,
                              double alpha, const double* A, int64_t lda, int64_t str_a,
                              double beta, double* C, int64_t ldc, int64_t str_c, int64_t batch);

/* Philox4x32-10: out[0..3] = philox(ctr[0..3], key[0..1]). */
void sbo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* Synthetic input streams (same mapping as the device generator):
 *   key = seed (lo, hi); counter = (block lo, block hi, stream, 0).
 *   f32 uniform [-1,1): element e uses block e/4, word e%4: (w>>8)*2^-23 - 1.
 *   f64 uniform [-1,1): element e uses block e/2, words 2(e%2), 2(e%2)+1:
 *                       ((w0>>5)*2^26 + (w1>>6)) * 2^-52 - 1.
 *   normal: element e uses block e/2; u1 = (53-bit from w0,w1 + 1)*2^-53 in
 *           (0,1], u2 = 53-bit from w2,w3 * 2^-53; Box-Muller in double,
 *           cos for even e, sin for odd e; times `scale`.             */
void sbo_fill_uniform_f32(float* out, int64_t n, uint64_t seed, uint32_t stream);
void sbo_fill_uniform_f64(double* out, int64_t n, uint64_t seed, uint32_t stream);
void sbo_fill_normal_f32(float* out, int64_t n, uint64_t seed, uint32_t stream, double scale);
void sbo_fill_normal_f64(double* out, int64_t n, uint64_t seed, uint32_t stream, double scale);

int sbo_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* SBO_H */
