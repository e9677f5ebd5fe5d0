// gemm_cfg_f32_256x128x16_w4x1.hip -- instantiates the float 256x128x16 MFMA tile
// (waves 4x1, prefetch depth 2, 2 wave(s) per SIMD: two workgroups per CU).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 256, 128, 16, 4, 1, 2, 2>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
