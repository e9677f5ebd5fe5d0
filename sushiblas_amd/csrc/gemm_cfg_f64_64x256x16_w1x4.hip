// gemm_cfg_f64_64x256x16_w1x4.hip -- instantiates the double 64x256x16 MFMA tile (waves 1x4).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<double, 64, 256, 16, 1, 4>(const GemmArgs<double>&, bool, bool,
                                                            bool, bool, int, hipStream_t);
}  // namespace sbx
