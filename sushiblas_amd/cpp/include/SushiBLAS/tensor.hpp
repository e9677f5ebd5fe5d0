// tensor.hpp -- strided view over a Storage (include/SushiBLAS/tensor.hpp:54-301
// of the reference): same fields, constructor semantics, views and quirks.
//
// Kept as in the reference (callers may depend on them):
//   * contiguous strides are computed from the layout in the constructor;
//   * the capacity check counts sizeof(float) per element (tensor.hpp:123);
//   * data() scales storage_offset by 8 bytes for FLOAT64 and 4 otherwise
//     (tensor.hpp:165).
// Changed, on purpose: reshape() and slice() keep the tensor's dtype (the
// reference rebuilds the view through the constructor and so resets it to
// FLOAT32, tensor.hpp:269/:299).
// Added for the HIP backend: device_data()/device_data_as<T>() give the
// address a kernel must use (data() is the host-visible one for SHARED).
// C++17: dimensions come as an initializer list, a vector, or pointer+rank
// instead of std::span.
#pragma once

#include <SushiBLAS/core/common.hpp>
#include <SushiBLAS/core/errors.hpp>
#include <SushiBLAS/storage.hpp>

#include <algorithm>
#include <array>
#include <cstdint>
#include <initializer_list>
#include <vector>

namespace SushiBLAS
{
    struct Tensor
    {
        std::array<int64_t, Core::MAX_TENSOR_RANK> shape{};
        std::array<int64_t, Core::MAX_TENSOR_RANK> strides{};
        int32_t rank = 0;
        Core::DataType dtype = Core::DataType::FLOAT32;
        Core::Layout layout = Core::Layout::ROW_MAJOR;
        int64_t num_elements = 0;
        SushiRuntime::sushi_ptr<Storage> storage;
        int64_t storage_offset = 0;

        Tensor() = default;

        Tensor(SushiRuntime::sushi_ptr<Storage> s, const int64_t* dims, int32_t n_dims,
               int64_t offset = 0, Core::Layout l = Core::Layout::ROW_MAJOR)
            : rank(n_dims), layout(l), storage(s), storage_offset(offset)
        {
            SB_THROW_IF(rank < 0 || static_cast<size_t>(rank) > Core::MAX_TENSOR_RANK,
                        "Rank {} exceeds limit of {}", rank, Core::MAX_TENSOR_RANK);
            int64_t elements = 1;
            if (layout == Core::Layout::ROW_MAJOR)
            {
                for (int i = rank - 1; i >= 0; --i)
                {
                    shape[i] = dims[i];
                    strides[i] = elements;
                    elements *= dims[i];
                }
            }
            else
            {
                for (int i = 0; i < rank; ++i)
                {
                    shape[i] = dims[i];
                    strides[i] = elements;
                    elements *= dims[i];
                }
            }
            num_elements = elements;
            if (storage)
            {
                SB_THROW_IF(storage_offset < 0, "Storage offset cannot be negative ({})", storage_offset);
                const size_t required = (static_cast<size_t>(num_elements) + storage_offset) * sizeof(float);
                SB_THROW_IF(required > storage->size_bytes,
                            "Storage capacity exceeded! Required: {} bytes, Available: {} bytes",
                            required, storage->size_bytes);
            }
        }

        Tensor(SushiRuntime::sushi_ptr<Storage> s, std::initializer_list<int64_t> dims,
               int64_t offset = 0, Core::Layout l = Core::Layout::ROW_MAJOR)
            : Tensor(s, dims.begin(), static_cast<int32_t>(dims.size()), offset, l) {}

        Tensor(SushiRuntime::sushi_ptr<Storage> s, const std::vector<int64_t>& dims,
               int64_t offset = 0, Core::Layout l = Core::Layout::ROW_MAJOR)
            : Tensor(s, dims.data(), static_cast<int32_t>(dims.size()), offset, l) {}

        /** @brief HIP device ordinal of the storage. */
        int get_device() const
        {
            SB_THROW_IF(!storage || !storage->allocator, "Tensor has no valid storage/allocator");
            return storage->allocator->get_device_of(storage->data_ptr);
        }

        size_t offset_bytes() const
        {
            const size_t element_size = (dtype == Core::DataType::FLOAT64) ? 8 : 4;
            return static_cast<size_t>(storage_offset) * element_size;
        }

        /** @brief Host-visible address (SHARED/HOST) or HBM address (DEVICE). */
        void* data() const
        {
            SB_THROW_IF(storage == nullptr, "Accessing data of a tensor with no storage");
            SB_THROW_IF(storage->data_ptr == nullptr, "Accessing data of a tensor with no data pointer");
            return static_cast<char*>(storage->data_ptr) + offset_bytes();
        }

        template <typename T = float>
        T* data_as() const { return static_cast<T*>(data()); }

        /** @brief Address a kernel uses for this view's first element. */
        void* device_data() const
        {
            SB_THROW_IF(storage == nullptr, "Accessing data of a tensor with no storage");
            SB_THROW_IF(storage->device_ptr == nullptr, "Tensor storage has no device address");
            return static_cast<char*>(storage->device_ptr) + offset_bytes();
        }

        template <typename T = float>
        T* device_data_as() const { return static_cast<T*>(device_data()); }

        bool is_contiguous() const
        {
            if (num_elements == 0) return true;
            int64_t expected = 1;
            if (layout == Core::Layout::ROW_MAJOR)
            {
                for (int i = rank - 1; i >= 0; --i)
                    if (shape[i] != 1)
                    {
                        if (strides[i] != expected) return false;
                        expected *= shape[i];
                    }
            }
            else
            {
                for (int i = 0; i < rank; ++i)
                    if (shape[i] != 1)
                    {
                        if (strides[i] != expected) return false;
                        expected *= shape[i];
                    }
            }
            return true;
        }

        bool is_aligned() const
        {
            return reinterpret_cast<uintptr_t>(data()) % SushiRuntime::Core::DEFAULT_ALIGNMENT == 0;
        }

        /** @brief View with dimensions dim0 and dim1 swapped (no data movement). */
        Tensor transpose(int32_t dim0, int32_t dim1) const
        {
            SB_THROW_IF(dim0 < 0 || dim1 < 0 || dim0 >= rank || dim1 >= rank,
                        "Invalid dimensions ({}, {}) for rank {}", dim0, dim1, rank);
            Tensor t = *this;
            std::swap(t.shape[dim0], t.shape[dim1]);
            std::swap(t.strides[dim0], t.strides[dim1]);
            return t;
        }

        /** @brief Same elements, new shape (contiguous tensors only). */
        Tensor reshape(std::initializer_list<int64_t> new_dims) const
        {
            int64_t n = 1;
            for (int64_t d : new_dims) n *= d;
            SB_THROW_IF(n != num_elements, "Element count mismatch. Current: {}, New: {}",
                        num_elements, n);
            SB_THROW_IF(!is_contiguous(), "Tensor must be contiguous for this operation");
            Tensor t(storage, new_dims, storage_offset, layout);
            t.dtype = dtype;
            return t;
        }

        /** @brief Sub-range [start, end) of dimension `dim` (negative indices wrap). */
        Tensor slice(int32_t dim, int64_t start, int64_t end) const
        {
            SB_THROW_IF(dim < 0 || dim >= rank, "Invalid dimension {}", dim);
            const int64_t size = shape[dim];
            if (start < 0) start += size;
            if (end < 0) end += size;
            start = std::max<int64_t>(0, std::min(start, size));
            end = std::max<int64_t>(start, std::min(end, size));
            std::array<int64_t, Core::MAX_TENSOR_RANK> dims = shape;
            dims[dim] = end - start;
            Tensor t(storage, dims.data(), rank, storage_offset + start * strides[dim], layout);
            t.dtype = dtype;
            return t;
        }
    };
} // namespace SushiBLAS
