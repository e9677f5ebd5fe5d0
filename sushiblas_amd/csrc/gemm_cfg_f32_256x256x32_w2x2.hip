// gemm_cfg_f32_256x256x32_w2x2.hip -- instantiates the float 256x256x32 MFMA tile
// (waves 2x2, prefetch depth 1, 1 wave(s) per SIMD).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 256, 256, 32, 2, 2, 1, 1>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
