// gemm_cfg_f32_256x64x16_w4x1.hip -- instantiates the float 256x64x16 MFMA tile (waves 4x1).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 256, 64, 16, 4, 1>(const GemmArgs<float>&, bool, bool,
                                                            bool, bool, int, hipStream_t);
}  // namespace sbx
