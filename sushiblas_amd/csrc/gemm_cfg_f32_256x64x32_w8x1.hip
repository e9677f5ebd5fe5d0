// gemm_cfg_f32_256x64x32_w8x1.hip -- instantiates the float 256x64x32 MFMA tile
// (waves 8x1, prefetch depth 2, 2 wave(s) per SIMD, v_mfma_f32_16x16x4_f32).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 256, 64, 32, 8, 1, 2, 2, 1>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
