// level3.hpp -- BLAS level-3 operations on the gfx950 backend
// (include/SushiBLAS/ops/blas/level3.hpp:50-117 of the reference).
// gemm and syrk keep the reference's signatures and contracts (trsm is not
// provided by this backend); the returned Event is a
// default (already complete) one, as the reference returns sycl::event()
// (src/ops/blas/level3/gemm.cpp:197): completion is observed through
// Engine::execute().
#pragma once

#include <SushiBLAS/tensor.hpp>
#include <SushiRuntime/SushiRuntime.h>

namespace SushiBLAS
{
    class Engine;

    class Level3
    {
        protected:
            explicit Level3(Engine& e) : engine_(e) {}
            Engine& engine_;

        public:
            /**
             * @brief C = alpha * op(A) * op(B) + beta * C, batched when rank > 2.
             *
             * m = C.shape[-2], n = C.shape[-1], k = transA ? A.shape[-2] : A.shape[-1];
             * leading dimensions come from the shapes (last dim for row-major,
             * second-to-last for column-major); batch = product of C's leading
             * dims with batch strides strides[-3]; the layout is A's.
             * FLOAT32 and FLOAT64 run on hand-written gfx950 MFMA kernels through
             * the C ABI (sbx_sgemm / sbx_dgemm and the strided-batched forms).
             * @throws std::runtime_error on rank < 2, dtype mismatch, or a dtype
             *         this backend does not run (HALF, COMPLEX*); a kernel-side
             *         failure throws from Engine::execute().
             */
            SushiRuntime::Execution::Event gemm(const Tensor& A, const Tensor& B, Tensor& C,
                                                bool transA = false, bool transB = false,
                                                float alpha = 1.0f, float beta = 0.0f);

            /**
             * @brief One triangle of C = alpha * op(A) * op(A)^T + beta * C
             *        (src/ops/blas/level3/syrk.cpp:84-194), batched when rank > 2.
             *
             * n = C.shape[-2] (C must be square); op(A) = A (n x k) when
             * !transA, A^T (A is k x n) when transA; `upper` selects the
             * triangle that is updated, the other is not touched.  lda/ldc from
             * the shapes, batch = product of C's leading dims with strides[-3],
             * layout from A.  FLOAT32 / FLOAT64 run the MFMA GEMM kernels over
             * the triangle's tiles only (sbx_ssyrk / sbx_dsyrk).
             * @throws std::runtime_error on rank < 2, dtype mismatch, non-square
             *         C, A not matching C, or HALF / COMPLEX tensors.
             */
            SushiRuntime::Execution::Event syrk(const Tensor& A, Tensor& C, bool upper = false,
                                                bool transA = false, float alpha = 1.0f,
                                                float beta = 0.0f);
    };
} // namespace SushiBLAS
