// gemm_cfg_f32_32x128x32_w1x4.hip -- instantiates the float 32x128x32 MFMA tile
// (waves 1x4, prefetch depth 2, 2 wave(s) per SIMD, v_mfma_f32_16x16x4_f32).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 32, 128, 32, 1, 4, 2, 2, 1>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
