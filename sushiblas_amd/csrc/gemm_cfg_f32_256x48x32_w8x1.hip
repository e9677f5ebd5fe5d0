// gemm_cfg_f32_256x48x32_w8x1.hip -- instantiates the float 256x64x32 MFMA tile
// computing its first 48 columns (waves 8x1, prefetch depth 2, 2 wave(s) per
// SIMD, v_mfma_f32_16x16x4_f32), for 32 < N <= 48.
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 256, 64, 32, 8, 1, 2, 2, 1, 48>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
