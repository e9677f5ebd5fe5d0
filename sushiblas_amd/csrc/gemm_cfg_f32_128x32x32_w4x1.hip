// gemm_cfg_f32_128x32x32_w4x1.hip -- instantiates the float 128x32x32 MFMA tile
// (waves 4x1, prefetch depth 2, 2 wave(s) per SIMD, v_mfma_f32_16x16x4_f32).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 128, 32, 32, 4, 1, 2, 2, 1>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
