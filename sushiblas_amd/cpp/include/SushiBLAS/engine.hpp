// engine.hpp -- entry point of SushiBLAS (include/SushiBLAS/engine.hpp:61-195,
// src/engine.cpp of the reference): owns the task graph and the default
// layout, creates tensors, exposes the BLAS ops, executes recorded work.
#pragma once

#include <SushiBLAS/core/common.hpp>
#include <SushiBLAS/core/errors.hpp>
#include <SushiBLAS/io.hpp>
#include <SushiBLAS/ops/blas.hpp>
#include <SushiBLAS/ops/math/nonlinear.hpp>
#include <SushiBLAS/storage.hpp>
#include <SushiBLAS/tensor.hpp>
#include <SushiRuntime/SushiRuntime.h>

#include <atomic>
#include <initializer_list>

namespace SushiBLAS
{
    class Engine
    {
        public:
            Engine(SushiRuntime::Execution::RuntimeContext& ctx,
                   Core::Layout layout = Core::Layout::ROW_MAJOR);

            Core::Layout get_layout() const { return default_layout_; }
            BLASOps blas() { return BLASOps(*this); }
            /** @brief Activations (engine.hpp:118 of the reference); relu only. */
            NonLinearOps nonlinear() { return NonLinearOps(*this); }
            /** @brief File IO (engine.hpp:88 of the reference): .npy and raw binary. */
            IO io() { return IO(*this); }

            SushiRuntime::Execution::RuntimeContext& get_context() { return context_; }
            SushiRuntime::Graph::TaskGraph& get_graph() { return graph_; }

            /** @brief Run every recorded task; the Event completes with them. */
            SushiRuntime::Execution::Event execute() { return graph_.execute(); }

            /** @brief New FLOAT32 tensor in the default layout. */
            Tensor create_tensor(std::initializer_list<int64_t> dims,
                                 SushiRuntime::Memory::AllocStrategy strat =
                                     SushiRuntime::Memory::AllocStrategy::SHARED);

            /** @brief New tensor of `dtype` (bytes per element: HALF 2, FLOAT32 4,
             *  FLOAT64 and COMPLEX32 8, COMPLEX64 16; src/engine.cpp:57-61). */
            Tensor create_tensor(std::initializer_list<int64_t> dims, Core::DataType dtype,
                                 SushiRuntime::Memory::AllocStrategy strat =
                                     SushiRuntime::Memory::AllocStrategy::SHARED);

            void set_seed(uint64_t s) { seed_ = s; }
            uint64_t get_seed() const { return seed_; }
            uint64_t get_and_increment_rng_offset() { return rng_offset_++; }

        private:
            SushiRuntime::Execution::RuntimeContext& context_;
            SushiRuntime::Graph::TaskGraph graph_;
            Core::Layout default_layout_;
            uint64_t seed_ = 0;
            std::atomic<uint64_t> rng_offset_{0};
    };
} // namespace SushiBLAS
