// nonlinear.hpp -- NonLinearOps on the gfx950 backend
// (include/SushiBLAS/ops/math/nonlinear.hpp of the reference).  Only relu is
// provided: it is the activation the reference's integration tests record
// after every GEMM (tests/runtime/test_framework_sim.cpp:51-57,109-110), and
// the one the task graph fuses into the GEMM epilogue.
#pragma once

#include <SushiBLAS/tensor.hpp>
#include <SushiRuntime/SushiRuntime.h>

namespace SushiBLAS
{
    class Engine;

    class NonLinearOps
    {
        public:
            explicit NonLinearOps(Engine& e) : engine_(e) {}

            /**
             * @brief In place: t[i] = t[i] > 0 ? t[i] : 0 over t.num_elements
             *        elements (src/ops/math/nonlinear/relu.cpp:38-41), so NaN and
             *        -0 become +0.  Recorded as "math.nonlinear.relu".
             *
             * The elements are the num_elements contiguous values starting at
             * the tensor's first element (storage base + storage_offset).  The
             * reference's kernel indexes from the storage base pointer
             * (nonlinear_internal.hpp:52,64) and so ignores storage_offset;
             * for offset-0 tensors, the only ones its tests use, the two agree.
             * When the task recorded just before it is a GEMM whose output is
             * exactly these elements, Engine::execute() runs the pair as one
             * fused kernel ("blas.lvl3.gemm+relu").
             * @throws std::runtime_error for HALF and COMPLEX tensors (FLOAT32
             *         and FLOAT64 only on this backend).
             */
            SushiRuntime::Execution::Event relu(Tensor& t);

        private:
            Engine& engine_;
    };
} // namespace SushiBLAS
