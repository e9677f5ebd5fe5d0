// engine.cpp -- Engine construction and tensor creation (src/engine.cpp:35-69
// of the reference, same byte sizes and storage path).
#include <SushiBLAS/engine.hpp>

namespace SushiBLAS
{
    Engine::Engine(SushiRuntime::Execution::RuntimeContext& ctx, Core::Layout layout)
        : context_(ctx), graph_(ctx), default_layout_(layout)
    {
    }

    Tensor Engine::create_tensor(std::initializer_list<int64_t> dims,
                                 SushiRuntime::Memory::AllocStrategy strat)
    {
        return create_tensor(dims, Core::DataType::FLOAT32, strat);
    }

    Tensor Engine::create_tensor(std::initializer_list<int64_t> dims, Core::DataType dtype,
                                 SushiRuntime::Memory::AllocStrategy strat)
    {
        size_t elements = 1;
        for (int64_t d : dims) elements *= static_cast<size_t>(d);
        size_t bpe = 4;
        if (dtype == Core::DataType::FLOAT64 || dtype == Core::DataType::COMPLEX32) bpe = 8;
        else if (dtype == Core::DataType::COMPLEX64) bpe = 16;
        else if (dtype == Core::DataType::HALF) bpe = 2;
        auto storage = SushiRuntime::make_sushi<Storage>(context_.get_allocator(), elements * bpe, strat);
        Tensor t(storage, dims, 0, default_layout_);
        t.dtype = dtype;
        return t;
    }
} // namespace SushiBLAS
