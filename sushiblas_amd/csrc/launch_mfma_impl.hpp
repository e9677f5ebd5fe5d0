// launch_mfma_impl.hpp -- definition of launch_mfma (see launch.hpp).  Only
// the gemm_cfg_*.hip translation units include this, each instantiating one
// tile configuration, so the configurations compile in parallel.
#pragma once

#include "launch.hpp"

namespace sbx {

template <typename T, int BM, int BN, int BK, int WM, int WN, int PF, int WPE, int MI, int BNC,
          int BMC>
hipError_t launch_mfma(const GemmArgs<T>& a, bool a_kc, bool b_kc, int batch, hipStream_t stream)
{
    const int tiles = a.tiles;
    const dim3 grid((unsigned)(a.num_full + (tiles - a.num_full) * a.split), 1, (unsigned)batch);
    const dim3 block(WM * WN * 64);
    // k-tail masking is compiled in only where a k-contiguous operand meets a
    // K that is not a multiple of the 16-byte vector (it costs 1-4 %)
    const bool tail = (a_kc || b_kc) && a.K % (16 / (int)sizeof(T)) != 0;
    // A grid one tile wide reads its operand once (see run() for when that
    // operand's loads go non-temporal); only the tall (BN <= 64) and wide
    // (BM <= 64) tiles, whose grids are that, compile the streaming form.
    constexpr int kStream = BN <= 64 ? 1 : (BM <= 64 ? 2 : 0);
    const bool streamed = kStream != 0 && a.stream_op == kStream;
#define SBX_LAUNCH(AK, BKC, TAIL)                                                                 \
    do {                                                                                          \
        if (streamed)                                                                             \
            gemm_mfma_kernel<T, BM, BN, BK, WM, WN, AK, BKC, TAIL, PF, WPE, MI, kStream, BNC, BMC>\
                <<<grid, block, 0, stream>>>(a);                                                  \
        else                                                                                      \
            gemm_mfma_kernel<T, BM, BN, BK, WM, WN, AK, BKC, TAIL, PF, WPE, MI, 0, BNC, BMC>      \
                <<<grid, block, 0, stream>>>(a);                                                  \
    } while (0)
    if (a_kc && b_kc) {
        if (tail) SBX_LAUNCH(true, true, true);
        else SBX_LAUNCH(true, true, false);
    } else if (a_kc) {
        if (tail) SBX_LAUNCH(true, false, true);
        else SBX_LAUNCH(true, false, false);
    } else if (b_kc) {
        if (tail) SBX_LAUNCH(false, true, true);
        else SBX_LAUNCH(false, true, false);
    } else {
        SBX_LAUNCH(false, false, false);
    }
#undef SBX_LAUNCH
    if (a.split > 1) {
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        // the reduction runs 256 threads per block whatever the tile's waves
        constexpr int CHUNKS = SplitReduce<T, BM, BN>::CHUNKS;
        const dim3 rgrid((unsigned)((tiles - a.num_full) * CHUNKS), 1, (unsigned)batch);
        splitk_reduce_kernel<T, BM, BN><<<rgrid, dim3(256), 0, stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace sbx
