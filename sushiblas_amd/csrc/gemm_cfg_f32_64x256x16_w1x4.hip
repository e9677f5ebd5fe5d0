// gemm_cfg_f32_64x256x16_w1x4.hip -- instantiates the float 64x256x16 MFMA tile (waves 1x4).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<float, 64, 256, 16, 1, 4>(const GemmArgs<float>&, bool, bool,
                                                            bool, bool, int, hipStream_t);
}  // namespace sbx
