// gemv.hpp -- row-major GEMV kernels (gemv.hip) and their launch plan.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sbx {

// Row-major problem: A is rows x cols with leading dimension lda.
//   trans == false: y[i] = alpha * sum_j A[i][j] x[j*incx] + beta * y[i*incy], i < rows
//   trans == true:  y[j] = alpha * sum_i A[i][j] x[i*incx] + beta * y[j*incy], j < cols
template <typename T>
struct GemvArgs {
    const T* A;
    const T* x;
    T* y;
    int64_t lda, incx, incy;
    int64_t rows, cols;
    T alpha, beta;
    int64_t cw;  // extent of one chunk of the reduction dimension
    T* ws;       // chunk partials (chunks x output length) when chunks > 1
};

struct GemvPlan {
    bool trans;
    bool vec;      // 16-byte loads of A (and of x for the rows kernel)
    int lanes;     // rows kernel: lanes per row; cols kernel: column threads per workgroup
    int64_t groups;  // grid.x
    int chunks;      // grid.y: ranges of the reduction dimension
    int64_t cw;      // extent of one range
    int64_t out_len;
};

template <typename T>
GemvPlan plan_gemv(bool trans, int64_t rows, int64_t cols, bool vec, int cus);

template <typename T>
hipError_t launch_gemv(GemvArgs<T> a, const GemvPlan& plan, hipStream_t stream);

}  // namespace sbx
