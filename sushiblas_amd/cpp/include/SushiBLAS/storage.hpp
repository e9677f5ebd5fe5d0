// storage.hpp -- reference-counted owner of one allocation
// (include/SushiBLAS/storage.hpp:49-113 of the reference).
//
// Same fields and behaviour: the size is rounded up to DEFAULT_ALIGNMENT
// (128 B), a zero-byte request or a null allocator throws, the destructor
// frees.  On HIP the allocation has two addresses:
//   data_ptr   -- what the reference exposes: host-visible for SHARED/HOST
//                 (tests fill tensors through it), the HBM address for DEVICE;
//   device_ptr -- the address kernels use (HBM for DEVICE/SHARED, the mapped
//                 address for HOST).
// copy_from_host / copy_to_host are the explicit staging helpers for DEVICE
// allocations (the reference's IO stages DEVICE tensors with queue.memcpy,
// src/io.cpp:73-78); SHARED allocations are staged by TaskGraph::execute().
#pragma once

#include <SushiBLAS/core/common.hpp>
#include <SushiBLAS/core/errors.hpp>
#include <SushiRuntime/SushiRuntime.h>

namespace SushiBLAS
{
    class alignas(64) Storage : public SushiRuntime::Core::RefCounted
    {
        public:
            void* data_ptr = nullptr;
            void* device_ptr = nullptr;
            size_t size_bytes = 0;
            size_t requested_bytes = 0;
            SushiRuntime::sushi_ptr<SushiRuntime::Memory::USMAllocator> allocator;
            SushiRuntime::Memory::AllocStrategy strategy;

            Storage(SushiRuntime::sushi_ptr<SushiRuntime::Memory::USMAllocator> alloc, size_t n_bytes,
                    SushiRuntime::Memory::AllocStrategy strat = SushiRuntime::Memory::AllocStrategy::SHARED)
                : requested_bytes(n_bytes), allocator(alloc), strategy(strat)
            {
                SB_THROW_IF(!allocator, "Allocator pointer cannot be null");
                SB_THROW_IF(n_bytes == 0, "Requested size cannot be zero");
                const size_t a = SushiRuntime::Core::DEFAULT_ALIGNMENT;
                size_bytes = (n_bytes + a - 1) / a * a;
                data_ptr = allocator->allocate(size_bytes, strategy);
                SB_THROW_IF(!data_ptr, "Allocation failed for {} bytes", size_bytes);
                device_ptr = allocator->device_address(data_ptr);
            }

            Storage(const Storage&) = delete;
            Storage& operator=(const Storage&) = delete;

            /** @brief Synchronous host -> allocation copy of `bytes` at byte `offset`. */
            void copy_from_host(const void* src, size_t bytes, size_t offset = 0)
            {
                SB_THROW_IF(offset + bytes > size_bytes, "copy of {} bytes at {} exceeds {} bytes",
                            bytes, offset, size_bytes);
                SB_THROW_IF(hipMemcpy(static_cast<char*>(device_ptr) + offset, src, bytes,
                                      hipMemcpyHostToDevice) != hipSuccess,
                            "hipMemcpy(H2D) failed");
                if (strategy == SushiRuntime::Memory::AllocStrategy::SHARED)
                    std::memcpy(static_cast<char*>(data_ptr) + offset, src, bytes);
            }

            /** @brief Synchronous allocation -> host copy of `bytes` at byte `offset`. */
            void copy_to_host(void* dst, size_t bytes, size_t offset = 0) const
            {
                SB_THROW_IF(offset + bytes > size_bytes, "copy of {} bytes at {} exceeds {} bytes",
                            bytes, offset, size_bytes);
                SB_THROW_IF(hipMemcpy(dst, static_cast<const char*>(device_ptr) + offset, bytes,
                                      hipMemcpyDeviceToHost) != hipSuccess,
                            "hipMemcpy(D2H) failed");
            }

        protected:
            ~Storage() override
            {
                if (data_ptr && allocator) allocator->deallocate(data_ptr);
            }
    };
} // namespace SushiBLAS
