// gemm_cfg_f32_64x64x32_w2x2.hip -- instantiates the float 64x64x32 MFMA tile
// (waves 2x2, prefetch depth 2, 2 wave(s) per SIMD, v_mfma_f32_32x32x2_f32).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 64, 64, 32, 2, 2, 2, 2>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
