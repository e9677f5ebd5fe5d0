// gemm_cfg_f32_256x256x32_w4x2.hip -- instantiates the float 256x256x32 MFMA tile
// (8 waves as 4x2, 64x128 each, prefetch depth 1, 2 waves per SIMD).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 256, 256, 32, 4, 2, 1, 2>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
