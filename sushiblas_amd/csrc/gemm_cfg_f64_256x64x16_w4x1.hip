// gemm_cfg_f64_256x64x16_w4x1.hip -- instantiates the double 256x64x16 MFMA tile (waves 4x1).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<double, 256, 64, 16, 4, 1>(const GemmArgs<double>&, bool, bool,
                                                            bool, bool, int, hipStream_t);
}  // namespace sbx
