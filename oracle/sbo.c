/*
 * sbo.c -- CPU oracle for the SushiBLAS GEMM hot path (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file's library; the product never links it.  The header (sbo.h) lists
 * the reference lines each function restates and what pins it.
 */
#include "sbo.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* Element accessors.  The reference passes (layout, trans, ld) straight to  */
/* oneMKL (gemm.cpp:45-51, :63/:76).  op(X)(r, c) of a matrix stored in      */
/* `layout` with leading dimension ld:                                       */
/*   stored index (sr, sc) = trans ? (c, r) : (r, c)                         */
/*   address = layout == row ? sr*ld + sc : sr + sc*ld                       */
/* ------------------------------------------------------------------------ */
static inline int64_t op_index(int layout, int trans, int64_t r, int64_t c, int64_t ld)
{
    int64_t sr = trans ? c : r;
    int64_t sc = trans ? r : c;
    return layout == 0 ? sr * ld + sc : sr + sc * ld;
}

static inline int64_t c_index(int layout, int64_t i, int64_t j, int64_t ldc)
{
    return layout == 0 ? i * ldc + j : i + j * ldc;
}

static int check_args(int layout, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                      int64_t ldc, int transA, int transB)
{
    if (layout != 0 && layout != 1) return 1;
    if (m < 0 || n < 0 || k < 0) return 1;
    /* minimum leading dimensions, as BLAS requires */
    int64_t a_rows = transA ? k : m, a_cols = transA ? m : k;
    int64_t b_rows = transB ? n : k, b_cols = transB ? k : n;
    int64_t need_a = layout == 0 ? a_cols : a_rows;
    int64_t need_b = layout == 0 ? b_cols : b_rows;
    int64_t need_c = layout == 0 ? n : m;
    if (lda < (need_a > 1 ? need_a : 1)) return 1;
    if (ldb < (need_b > 1 ? need_b : 1)) return 1;
    if (ldc < (need_c > 1 ? need_c : 1)) return 1;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Blocked GEMM.  Each OpenMP task owns one MC x NC block of C across the   */
/* whole k range, packs op(A) into MR-row panels and op(B) into NR-column    */
/* panels (both k-major) and runs an MR x NR register micro-kernel.          */
/* ------------------------------------------------------------------------ */
#define MC 64
#define NC 256
#define KC 256

#define DEFINE_BLOCKED(NAME, T, ACC, MR, NR)                                                   \
_Static_assert(MC % (MR) == 0 && NC % (NR) == 0, "packing buffers assume MR | MC, NR | NC");  \
static void NAME##_micro(int64_t kc, const ACC* restrict ap, const ACC* restrict bp,          \
                         ACC* restrict c, int64_t ldcw)                                        \
{                                                                                              \
    ACC r[MR][NR];                                                                             \
    for (int i = 0; i < MR; ++i)                                                               \
        for (int j = 0; j < NR; ++j) r[i][j] = 0;                                              \
    for (int64_t p = 0; p < kc; ++p) {                                                         \
        const ACC* b = bp + p * NR;                                                            \
        for (int i = 0; i < MR; ++i) {                                                         \
            ACC a = ap[p * MR + i];                                                            \
            for (int j = 0; j < NR; ++j) r[i][j] += a * b[j];                                  \
        }                                                                                      \
    }                                                                                          \
    for (int i = 0; i < MR; ++i)                                                               \
        for (int j = 0; j < NR; ++j) c[i * ldcw + j] += r[i][j];                               \
}                                                                                              \
                                                                                               \
static void NAME(int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,         \
                 ACC alpha, const T* A, int64_t lda, const T* B, int64_t ldb, ACC beta, T* C,  \
                 int64_t ldc)                                                                  \
{                                                                                              \
    const int64_t mblocks = (m + MC - 1) / MC, nblocks = (n + NC - 1) / NC;                   \
    const int64_t ntiles = mblocks * nblocks;                                                  \
    _Pragma("omp parallel")                                                                    \
    {                                                                                          \
        ACC* ap = (ACC*)aligned_alloc(64, sizeof(ACC) * MC * KC);                              \
        ACC* bp = (ACC*)aligned_alloc(64, sizeof(ACC) * KC * NC);                              \
        ACC* acc = (ACC*)aligned_alloc(64, sizeof(ACC) * MC * NC);                             \
        _Pragma("omp for schedule(dynamic, 1)")                                                \
        for (int64_t t = 0; t < ntiles; ++t) {                                                 \
            const int64_t i0 = (t / nblocks) * MC, j0 = (t % nblocks) * NC;                    \
            const int64_t mc = m - i0 < MC ? m - i0 : MC;                                      \
            const int64_t nc = n - j0 < NC ? n - j0 : NC;                                      \
            const int64_t mcp = (mc + MR - 1) / MR * MR, ncp = (nc + NR - 1) / NR * NR;        \
            memset(acc, 0, sizeof(ACC) * MC * NC);                                             \
            for (int64_t p0 = 0; p0 < k; p0 += KC) {                                           \
                const int64_t kc = k - p0 < KC ? k - p0 : KC;                                  \
                for (int64_t ir = 0; ir < mcp; ir += MR)                                       \
                    for (int64_t p = 0; p < kc; ++p)                                           \
                        for (int i = 0; i < MR; ++i) {                                         \
                            int64_t gi = i0 + ir + i;                                          \
                            ap[ir * kc + p * MR + i] = gi < m                                  \
                                ? (ACC)A[op_index(layout, transA, gi, p0 + p, lda)] : (ACC)0;  \
                        }                                                                      \
                for (int64_t jr = 0; jr < ncp; jr += NR)                                       \
                    for (int64_t p = 0; p < kc; ++p)                                           \
                        for (int j = 0; j < NR; ++j) {                                         \
                            int64_t gj = j0 + jr + j;                                          \
                            bp[jr * kc + p * NR + j] = gj < n                                  \
                                ? (ACC)B[op_index(layout, transB, p0 + p, gj, ldb)] : (ACC)0;  \
                        }                                                                      \
                for (int64_t jr = 0; jr < ncp; jr += NR)                                       \
                    for (int64_t ir = 0; ir < mcp; ir += MR)                                   \
                        NAME##_micro(kc, ap + ir * kc, bp + jr * kc, acc + ir * NC + jr, NC);  \
            }                                                                                  \
            for (int64_t i = 0; i < mc; ++i)                                                   \
                for (int64_t j = 0; j < nc; ++j) {                                             \
                    T* cp = C + c_index(layout, i0 + i, j0 + j, ldc);                          \
                    ACC v = alpha * acc[i * NC + j];                                           \
                    if (beta != (ACC)0) v += beta * (ACC)(*cp);                                \
                    *cp = (T)v;                                                                \
                }                                                                              \
        }                                                                                      \
        free(ap);                                                                              \
        free(bp);                                                                              \
        free(acc);                                                                             \
    }                                                                                          \
}

DEFINE_BLOCKED(blocked_f32_f32, float, float, 4, 8)
DEFINE_BLOCKED(blocked_f32_f64, float, double, 4, 8)
DEFINE_BLOCKED(blocked_f64_f64, double, double, 4, 8)

/* C <- beta*C over the m x n window (beta == 0 writes zeros, never reads C). */
#define DEFINE_SCALE(NAME, T)                                                                  \
static void NAME(int layout, int64_t m, int64_t n, T beta, T* C, int64_t ldc)                 \
{                                                                                              \
    _Pragma("omp parallel for")                                                                \
    for (int64_t i = 0; i < m; ++i)                                                            \
        for (int64_t j = 0; j < n; ++j) {                                                      \
            T* cp = C + c_index(layout, i, j, ldc);                                            \
            *cp = beta == (T)0 ? (T)0 : beta * *cp;                                            \
        }                                                                                      \
}
DEFINE_SCALE(scale_f32, float)
DEFINE_SCALE(scale_f64, double)

int sbo_sgemm_strided_batched(int layout, int transA, int transB, int64_t m, int64_t n,
                              int64_t k, float alpha, const float* A, int64_t lda,
                              int64_t str_a, const float* B, int64_t ldb, int64_t str_b,
                              float beta, float* C, int64_t ldc, int64_t str_c,
                              int64_t batch, int acc_mode)
{
    if (check_args(layout, m, n, k, lda, ldb, ldc, transA, transB) || batch < 0) return 1;
    if (m == 0 || n == 0) return 0;
    for (int64_t b = 0; b < batch; ++b) {
        const float* a = A + b * str_a;
        const float* bb = B + b * str_b;
        float* c = C + b * str_c;
        if (alpha == 0.0f || k == 0) { scale_f32(layout, m, n, beta, c, ldc); continue; }
        if (acc_mode == 1)
            blocked_f32_f64(layout, transA, transB, m, n, k, (double)alpha, a, lda, bb, ldb,
                            (double)beta, c, ldc);
        else
            blocked_f32_f32(layout, transA, transB, m, n, k, alpha, a, lda, bb, ldb, beta, c, ldc);
    }
    return 0;
}

int sbo_dgemm_strided_batched(int layout, int transA, int transB, int64_t m, int64_t n,
                              int64_t k, double alpha, const double* A, int64_t lda,
                              int64_t str_a, const double* B, int64_t ldb, int64_t str_b,
                              double beta, double* C, int64_t ldc, int64_t str_c,
                              int64_t batch, int acc_mode)
{
    (void)acc_mode;
    if (check_args(layout, m, n, k, lda, ldb, ldc, transA, transB) || batch < 0) return 1;
    if (m == 0 || n == 0) return 0;
    for (int64_t b = 0; b < batch; ++b) {
        const double* a = A + b * str_a;
        const double* bb = B + b * str_b;
        double* c = C + b * str_c;
        if (alpha == 0.0 || k == 0) { scale_f64(layout, m, n, beta, c, ldc); continue; }
        blocked_f64_f64(layout, transA, transB, m, n, k, alpha, a, lda, bb, ldb, beta, c, ldc);
    }
    return 0;
}

int sbo_sgemm(int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
              float beta, float* C, int64_t ldc, int acc_mode)
{
    return sbo_sgemm_strided_batched(layout, transA, transB, m, n, k, alpha, A, lda, 0, B, ldb,
                                     0, beta, C, ldc, 0, 1, acc_mode);
}

int sbo_dgemm(int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              double alpha, const double* A, int64_t lda, const double* B, int64_t ldb,
              double beta, double* C, int64_t ldc, int acc_mode)
{
    return sbo_dgemm_strided_batched(layout, transA, transB, m, n, k, alpha, A, lda, 0, B, ldb,
                                     0, beta, C, ldc, 0, 1, acc_mode);
}

/* ------------------------------------------------------------------------ */
/* Independent brute force: no packing, no blocking, long double.            */
/* ------------------------------------------------------------------------ */
int sbo_gemm_naive_ld(int elem, int layout, int transA, int transB, int64_t m, int64_t n,
                      int64_t k, double alpha, const void* A, int64_t lda, const void* B,
                      int64_t ldb, double beta, void* C, int64_t ldc)
{
    if (elem != 4 && elem != 8) return 2;
    if (check_args(layout, m, n, k, lda, ldb, ldc, transA, transB)) return 1;
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            long double s = 0.0L;
            if (alpha != 0.0)
                for (int64_t p = 0; p < k; ++p) {
                    int64_t ia = op_index(layout, transA, i, p, lda);
                    int64_t ib = op_index(layout, transB, p, j, ldb);
                    long double a = elem == 4 ? (long double)((const float*)A)[ia]
                                              : (long double)((const double*)A)[ia];
                    long double b = elem == 4 ? (long double)((const float*)B)[ib]
                                              : (long double)((const double*)B)[ib];
                    s += a * b;
                }
            int64_t ic = c_index(layout, i, j, ldc);
            long double v = (long double)alpha * s;
            if (beta != 0.0)
                v += (long double)beta * (elem == 4 ? (long double)((float*)C)[ic]
                                                    : (long double)((double*)C)[ic]);
            if (elem == 4) ((float*)C)[ic] = (float)v;
            else ((double*)C)[ic] = (double)v;
        }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Normwise relative Frobenius error.                                        */
/* ------------------------------------------------------------------------ */
#define DEFINE_ERR(NAME, T)                                                                    \
double NAME(int64_t rows, int64_t cols, const T* X, int64_t ldx, const T* Y, int64_t ldy)     \
{                                                                                              \
    double num = 0.0, den = 0.0;                                                               \
    _Pragma("omp parallel for reduction(+ : num, den)")                                        \
    for (int64_t i = 0; i < rows; ++i)                                                         \
        for (int64_t j = 0; j < cols; ++j) {                                                   \
            double y = (double)Y[i * ldy + j];                                                 \
            double d = (double)X[i * ldx + j] - y;                                             \
            num += d * d;                                                                      \
            den += y * y;                                                                      \
        }                                                                                      \
    if (den == 0.0) return num == 0.0 ? 0.0 : INFINITY;                                        \
    return sqrt(num / den);                                                                    \
}
DEFINE_ERR(sbo_rel_fro_err_f32, float)
DEFINE_ERR(sbo_rel_fro_err_f64, double)

/* ------------------------------------------------------------------------ */
/* ReLU (relu.cpp:38-41).                                                    */
/* ------------------------------------------------------------------------ */
void sbo_relu_f32(float* x, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

void sbo_relu_f64(double* x, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] > 0.0 ? x[i] : 0.0;
}

/* ------------------------------------------------------------------------ */
/* GEMV (gemv.cpp:44-61 -> oneMKL {row,column}_major::gemv).  op(A) is      */
/* ylen x xlen with ylen = trans ? n : m; each y element is one dot product  */
/* in double, in index order, then alpha and beta in double and one rounding */
/* to T.  Netlib quick returns: m == 0 || n == 0 leaves y alone; alpha == 0  */
/* gives y = beta*y (beta == 0: zeros, y not read).                          */
/* ------------------------------------------------------------------------ */
#define DEFINE_GEMV(NAME, T)                                                                      \
int NAME(int layout, int trans, int64_t m, int64_t n, T alpha, const T* A, int64_t lda,          \
         const T* x, int64_t incx, T beta, T* y, int64_t incy)                                   \
{                                                                                                 \
    if (layout != 0 && layout != 1) return 1;                                                     \
    if (m < 0 || n < 0 || incx <= 0 || incy <= 0) return 1;                                       \
    const int64_t need = layout == 0 ? n : m;                                                     \
    if (lda < (need > 1 ? need : 1)) return 1;                                                    \
    if (m == 0 || n == 0) return 0;                                                               \
    const int64_t ylen = trans ? n : m, xlen = trans ? m : n;                                     \
    if (alpha == (T)0) {                                                                          \
        if (beta == (T)1) return 0;                                                               \
        for (int64_t i = 0; i < ylen; ++i)                                                        \
            y[i * incy] = beta == (T)0 ? (T)0 : (T)((double)beta * (double)y[i * incy]);          \
        return 0;                                                                                 \
    }                                                                                             \
    /* op(A)(i, j) is contiguous along j for row-major A or column-major A^T; */ \
    /* otherwise along i, and the loops are interchanged over blocks of 256   */ \
    /* outputs -- each output still sums over j in increasing order.          */ \
    const int along_j = (layout == 0) == (trans == 0);                                            \
    _Pragma("omp parallel for schedule(static)")                                                  \
    for (int64_t i0 = 0; i0 < ylen; i0 += 256) {                                                  \
        const int64_t i1 = i0 + 256 < ylen ? i0 + 256 : ylen;                                     \
        double s[256];                                                                            \
        for (int64_t i = i0; i < i1; ++i) s[i - i0] = 0.0;                                        \
        if (along_j) {                                                                            \
            for (int64_t i = i0; i < i1; ++i)                                                     \
                for (int64_t j = 0; j < xlen; ++j)                                                \
                    s[i - i0] += (double)A[op_index(layout, trans, i, j, lda)] *                  \
                                 (double)x[j * incx];                                             \
        } else {                                                                                  \
            for (int64_t j = 0; j < xlen; ++j) {                                                  \
                const double xj = (double)x[j * incx];                                            \
                for (int64_t i = i0; i < i1; ++i)                                                 \
                    s[i - i0] += (double)A[op_index(layout, trans, i, j, lda)] * xj;              \
            }                                                                                     \
        }                                                                                         \
        for (int64_t i = i0; i < i1; ++i) {                                                       \
            double v = (double)alpha * s[i - i0];                                                 \
            if (beta != (T)0) v += (double)beta * (double)y[i * incy];                            \
            y[i * incy] = (T)v;                                                                   \
        }                                                                                         \
    }                                                                                             \
    return 0;                                                                                     \
}
DEFINE_GEMV(sbo_sgemv, float)
DEFINE_GEMV(sbo_dgemv, double)

/* ------------------------------------------------------------------------ */
/* SYRK (syrk.cpp:44-77 -> oneMKL {row,column}_major::syrk[_batch]).  op(A) */
/* is n x k (trans ? A^T : A); for (i, j) in the requested triangle          */
/* (upper: j >= i, lower: j <= i) C(i, j) = alpha * sum_l op(A)(i, l)        */
/* op(A)(j, l) + beta * C(i, j), the sum in double in index order; the other */
/* triangle is never touched.  alpha == 0 || k == 0: C = beta*C on the      */
/* triangle; beta == 0: C not read.                                          */
/* ------------------------------------------------------------------------ */
#define DEFINE_SYRK(NAME, T)                                                                      \
int NAME(int layout, int upper, int trans, int64_t n, int64_t k, T alpha, const T* A,            \
         int64_t lda, int64_t str_a, T beta, T* C, int64_t ldc, int64_t str_c, int64_t batch)    \
{                                                                                                 \
    if (layout != 0 && layout != 1) return 1;                                                     \
    if (n < 0 || k < 0 || batch < 0) return 1;                                                    \
    const int64_t a_rows = trans ? k : n, a_cols = trans ? n : k;                                 \
    const int64_t need_a = layout == 0 ? a_cols : a_rows;                                         \
    if (lda < (need_a > 1 ? need_a : 1) || ldc < (n > 1 ? n : 1)) return 1;                       \
    const int quick = alpha == (T)0 || k == 0;                                                    \
    /* op(A) copied into rows of doubles (exact), so every dot product reads */ \
    /* contiguous memory whatever the layout and transpose                    */ \
    double* rows = quick || n == 0 ? NULL : (double*)malloc((size_t)n * (size_t)k * sizeof(double)); \
    if (!quick && n > 0 && !rows) return 2;                                                       \
    for (int64_t b = 0; b < batch; ++b) {                                                         \
        const T* a = A + b * str_a;                                                               \
        T* c = C + b * str_c;                                                                     \
        if (rows) {                                                                               \
            _Pragma("omp parallel for schedule(static)")                                          \
            for (int64_t i = 0; i < n; ++i)                                                       \
                for (int64_t l = 0; l < k; ++l)                                                   \
                    rows[i * k + l] = (double)a[op_index(layout, trans, i, l, lda)];              \
        }                                                                                         \
        _Pragma("omp parallel for schedule(dynamic, 8)")                                          \
        for (int64_t i = 0; i < n; ++i) {                                                         \
            const int64_t j0 = upper ? i : 0, j1 = upper ? n : i + 1;                             \
            for (int64_t j = j0; j < j1; ++j) {                                                   \
                T* cp = c + c_index(layout, i, j, ldc);                                           \
                double v = 0.0;                                                                   \
                if (!quick) {                                                                     \
                    const double* ri = rows + i * k;                                              \
                    const double* rj = rows + j * k;                                              \
                    double s = 0.0;                                                               \
                    for (int64_t l = 0; l < k; ++l) s += ri[l] * rj[l];                           \
                    v = (double)alpha * s;                                                        \
                }                                                                                 \
                if (beta != (T)0) v += (double)beta * (double)*cp;                                \
                *cp = (T)v;                                                                       \
            }                                                                                     \
        }                                                                                         \
    }                                                                                             \
    free(rows);                                                                                   \
    return 0;                                                                                     \
}
DEFINE_SYRK(sbo_ssyrk_strided_batched, float)
DEFINE_SYRK(sbo_dsyrk_strided_batched, double)

/* ------------------------------------------------------------------------ */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11).                        */
/* ------------------------------------------------------------------------ */
void sbo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static inline void block_words(uint64_t seed, uint32_t stream, uint64_t block, uint32_t w[4])
{
    uint32_t ctr[4] = {(uint32_t)block, (uint32_t)(block >> 32), stream, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    sbo_philox4x32_10(ctr, key, w);
}

void sbo_fill_uniform_f32(float* out, int64_t n, uint64_t seed, uint32_t stream)
{
    _Pragma("omp parallel for")
    for (int64_t b = 0; b < (n + 3) / 4; ++b) {
        uint32_t w[4];
        block_words(seed, stream, (uint64_t)b, w);
        for (int t = 0; t < 4 && 4 * b + t < n; ++t)
            out[4 * b + t] = (float)(w[t] >> 8) * 0x1p-23f - 1.0f;
    }
}

static inline double u53(uint32_t a, uint32_t b)
{
    return (double)(((uint64_t)(a >> 5) << 26) | (uint64_t)(b >> 6));
}

void sbo_fill_uniform_f64(double* out, int64_t n, uint64_t seed, uint32_t stream)
{
    _Pragma("omp parallel for")
    for (int64_t b = 0; b < (n + 1) / 2; ++b) {
        uint32_t w[4];
        block_words(seed, stream, (uint64_t)b, w);
        for (int t = 0; t < 2 && 2 * b + t < n; ++t)
            out[2 * b + t] = u53(w[2 * t], w[2 * t + 1]) * 0x1p-52 - 1.0;
    }
}

static inline void normal_pair(uint64_t seed, uint32_t stream, uint64_t b, double* z0, double* z1)
{
    uint32_t w[4];
    block_words(seed, stream, b, w);
    double u1 = (u53(w[0], w[1]) + 1.0) * 0x1p-53; /* (0, 1] */
    double u2 = u53(w[2], w[3]) * 0x1p-53;         /* [0, 1) */
    double r = sqrt(-2.0 * log(u1));
    double th = 6.283185307179586476925286766559 * u2;
    *z0 = r * cos(th);
    *z1 = r * sin(th);
}

void sbo_fill_normal_f32(float* out, int64_t n, uint64_t seed, uint32_t stream, double scale)
{
    _Pragma("omp parallel for")
    for (int64_t b = 0; b < (n + 1) / 2; ++b) {
        double z0, z1;
        normal_pair(seed, stream, (uint64_t)b, &z0, &z1);
        out[2 * b] = (float)(z0 * scale);
        if (2 * b + 1 < n) out[2 * b + 1] = (float)(z1 * scale);
    }
}

void sbo_fill_normal_f64(double* out, int64_t n, uint64_t seed, uint32_t stream, double scale)
{
    _Pragma("omp parallel for")
    for (int64_t b = 0; b < (n + 1) / 2; ++b) {
        double z0, z1;
        normal_pair(seed, stream, (uint64_t)b, &z0, &z1);
        out[2 * b] = z0 * scale;
        if (2 * b + 1 < n) out[2 * b + 1] = z1 * scale;
    }
}

int sbo_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
