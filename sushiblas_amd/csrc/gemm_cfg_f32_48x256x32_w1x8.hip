// gemm_cfg_f32_48x256x32_w1x8.hip -- instantiates the float 64x256x32 MFMA tile
// computing its first 48 rows (waves 1x8, prefetch depth 2, 2 wave(s) per
// SIMD, v_mfma_f32_16x16x4_f32), for 32 < M <= 48.
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 64, 256, 32, 1, 8, 2, 2, 1, 256, 48>(
    const GemmArgs<float>&, bool, bool, int, hipStream_t);
}  // namespace sbx
