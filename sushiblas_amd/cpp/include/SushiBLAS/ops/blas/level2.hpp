// level2.hpp -- BLAS level-2 operations on the gfx950 backend
// (include/SushiBLAS/ops/blas/level2.hpp:48-70 of the reference).  gemv keeps
// the reference's signature and contract; the other level-2 routines are not
// provided by this backend.
#pragma once

#include <SushiBLAS/tensor.hpp>
#include <SushiRuntime/SushiRuntime.h>

namespace SushiBLAS
{
    class Engine;

    class Level2
    {
        protected:
            explicit Level2(Engine& e) : engine_(e) {}
            Engine& engine_;

        public:
            /**
             * @brief y = alpha * op(A) * x + beta * y (src/ops/blas/level2/gemv.cpp:65-148).
             *
             * m = A.shape[-2], n = A.shape[-1] (leading dims of a higher-rank A
             * are ignored: no batching, gemv.cpp:75); lda from the shape and A's
             * layout; x and y are vectors of transA ? (m, n) : (n, m) elements,
             * stride 1 when contiguous, else a rank-1 tensor's stride
             * (utils.hpp:47-60).  FLOAT32 and FLOAT64 run on the gfx950 GEMV
             * kernels through sbx_sgemv / sbx_dgemv.
             * @throws std::runtime_error on rank < 2, dtype mismatch, vector
             *         length mismatch, a non-contiguous vector of rank > 1, or a
             *         dtype this backend does not run (HALF, COMPLEX*).
             */
            SushiRuntime::Execution::Event gemv(const Tensor& A, const Tensor& x, Tensor& y,
                                                bool transA = false, float alpha = 1.0f,
                                                float beta = 0.0f);
    };
} // namespace SushiBLAS
