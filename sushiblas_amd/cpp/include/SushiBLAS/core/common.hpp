// common.hpp -- enums and limits of the SushiBLAS data model
// (include/SushiBLAS/core/common.hpp:41-59 of the reference: same names and values).
#pragma once

#include <cstddef>
#include <cstdint>

namespace SushiBLAS
{
    namespace Core
    {
        /** @brief Memory layout of a tensor. */
        enum class Layout : uint8_t
        {
            ROW_MAJOR,
            COLUMN_MAJOR
        };

        /** @brief Element types.  The gfx950 GEMM path runs FLOAT32 and FLOAT64. */
        enum class DataType : uint8_t
        {
            HALF,
            FLOAT32,
            FLOAT64,
            COMPLEX32,
            COMPLEX64
        };

        /** @brief Maximum tensor rank. */
        inline constexpr size_t MAX_TENSOR_RANK = 6;
    } // namespace Core
} // namespace SushiBLAS

namespace sb = SushiBLAS;
