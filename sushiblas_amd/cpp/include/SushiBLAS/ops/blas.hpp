// blas.hpp -- BLASOps facade (include/SushiBLAS/ops/blas.hpp:49-57 of the
// reference).  This backend provides level-2 gemv and level-3 gemm / syrk.
#pragma once

#include <SushiBLAS/ops/blas/level2.hpp>
#include <SushiBLAS/ops/blas/level3.hpp>

namespace SushiBLAS
{
    class BLASOps : public Level2, public Level3
    {
        public:
            explicit BLASOps(Engine& e) : Level2(e), Level3(e) {}
    };
} // namespace SushiBLAS
