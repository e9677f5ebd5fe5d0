// level3.hpp -- BLAS level-3 operations on the gfx950 backend
// (include/SushiBLAS/ops/blas/level3.hpp:50-117 of the reference).
// gemm keeps the reference's signature and contract; the returned Event is a
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
    };
} // namespace SushiBLAS
