// gemm_cfg_f32_128x128x16_w2x2.hip -- instantiates the float 128x128x16 MFMA tile
// (waves 2x2, prefetch depth 2, 2 wave(s) per SIMD).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 128, 128, 16, 2, 2, 2, 2>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
