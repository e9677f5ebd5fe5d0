// blas.hpp -- BLASOps facade (include/SushiBLAS/ops/blas.hpp:49-57 of the
// reference).  This backend provides the level-3 GEMM only.
#pragma once

#include <SushiBLAS/ops/blas/level3.hpp>

namespace SushiBLAS
{
    class BLASOps : public Level3
    {
        public:
            explicit BLASOps(Engine& e) : Level3(e) {}
    };
} // namespace SushiBLAS
