// gemm_cfg_f32_64x128x32_w2x2.hip -- instantiates the float 64x128x32 MFMA tile
// (waves 2x2, prefetch depth 2, 2 wave(s) per SIMD).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 64, 128, 32, 2, 2, 2, 2>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
