// launch.hpp -- host-side launchers for the GEMM kernels.
//
// launch_mfma<T, BM, BN, BK, WAVES_M, WAVES_N, PF, WPE, MI> picks one of the 7
// compiled variants (A k-contiguous or not, B k-contiguous or not, and for a
// k-contiguous operand whether K needs tail masking) and launches it on
// `stream`.
#pragma once

#include <hip/hip_runtime.h>

#include "gemm_mfma.hpp"

namespace sbx {

template <typename T, int BM, int BN, int BK, int WM, int WN, int PF, int WPE, int MI = 0,
          int BNC = BN, int BMC = BM>
hipError_t launch_mfma(const GemmArgs<T>& a, bool a_kc, bool b_kc, int batch, hipStream_t stream);

// One-launch GEMM for small problems (gemm_small.hip): 32x32 tiles of C,
// the `waves` (4, or 8 for fp32) waves of a workgroup cutting K that many ways;
// a.tiles_m/tiles_n count 32-wide tiles.
template <typename T>
hipError_t launch_small(const GemmArgs<T>& a, bool a_kc, bool b_kc, int batch, hipStream_t stream,
                        int waves);

// Generic (non-MFMA) fallback: 64x64 tiles, 64-bit addressing, any ld.
template <typename T>
hipError_t launch_generic(const GemmArgs<T>& a, bool trans_a, bool trans_b, int batch,
                          hipStream_t stream);

// C <- beta*C (beta == 0 stores zeros without reading C), then ReLU if relu;
// uplo 1 / 2: only the lower / upper triangle; with a grouped-launch table,
// entry z's C is table[3z + 2].
template <typename T>
hipError_t launch_scale(T* C, int64_t ldc, int64_t str_c, int64_t m, int64_t n, T beta,
                        int relu, int uplo, int batch, hipStream_t stream,
                        const void* const* table = nullptr);

// x <- max(x, 0) elementwise (NaN -> 0) over n contiguous elements.
template <typename T>
hipError_t launch_relu(T* x, int64_t n, hipStream_t stream);

// Tile configurations compiled into the library, one translation unit each
// (gemm_cfg_*.hip instantiates launch_mfma from launch_mfma_impl.hpp):
// (T, BM, BN, BK, waves along M, waves along N, prefetch depth, waves/SIMD,
// MFMA shape: 0 = 32x32x2 for fp32 / 16x16x4 for fp64, 1 = 16x16x4 fp32)
#define SBX_MFMA_CONFIGS(X)  \
    X(float, 256, 256, 32, 4, 2, 1, 2, 0) \
    X(float, 256, 128, 16, 4, 1, 2, 2, 0) \
    X(float, 128, 128, 16, 2, 2, 2, 2, 0) \
    X(float, 128, 128, 16, 2, 2, 2, 3, 0) \
    X(float, 128, 64, 32, 2, 2, 2, 2, 0) \
    X(float, 256, 64, 32, 8, 1, 2, 2, 1) \
    X(float, 64, 128, 32, 2, 2, 2, 2, 0) \
    X(float, 64, 256, 32, 1, 8, 2, 2, 1) \
    X(float, 128, 32, 32, 4, 1, 2, 2, 1) \
    X(float, 32, 128, 32, 1, 4, 2, 2, 1) \
    X(float, 64, 64, 32, 2, 2, 2, 2, 0) \
    X(double, 128, 128, 16, 2, 2, 1, 2, 0) \
    X(double, 128, 64, 16, 2, 2, 2, 2, 0) \
    X(double, 64, 128, 16, 2, 2, 2, 2, 0) \
    X(double, 64, 64, 16, 2, 2, 2, 2, 0)

#define SBX_EXTERN_LAUNCH(T, BM, BN, BK, WM, WN, PF, WPE, MI)                                    \
    extern template hipError_t launch_mfma<T, BM, BN, BK, WM, WN, PF, WPE, MI>(                     \
        const GemmArgs<T>&, bool, bool, int, hipStream_t);
SBX_MFMA_CONFIGS(SBX_EXTERN_LAUNCH)
#undef SBX_EXTERN_LAUNCH

}  // namespace sbx
