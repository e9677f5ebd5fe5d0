// gemm_cfg_f64_64x64x16_w2x2.hip -- instantiates the double 64x64x16 MFMA tile
// (waves 2x2, prefetch depth 2, 2 wave(s) per SIMD, v_mfma_f64_16x16x4_f64).
#include "launch_mfma_impl.hpp"

namespace sbx {
template hipError_t launch_mfma<double, 64, 64, 16, 2, 2, 2, 2>(
    const GemmArgs<double>&, bool, bool, int, hipStream_t);
}  // namespace sbx
