// gemm_cfg_f32_128x128x16_w2x2_o3.hip -- instantiates the float 128x128x16 MFMA tile
// (waves 2x2, prefetch depth 2) compiled for 3 waves per SIMD: at most 168
// VGPRs, so three workgroups share a CU (768 tiles in one round on 256 CUs).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 128, 128, 16, 2, 2, 2, 3>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
