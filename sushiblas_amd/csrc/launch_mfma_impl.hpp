// launch_mfma_impl.hpp -- definition of launch_mfma (see launch.hpp).  Only
// the gemm_cfg_*.hip translation units include this, each instantiating one
// tile configuration, so the 16 kernel variants per configuration compile in
// parallel.
#pragma once

#include "launch.hpp"

namespace sbx {

template <typename T, int BM, int BN, int BK, int WM, int WN, int PF, int WPE>
hipError_t launch_mfma(const GemmArgs<T>& a, bool a_kc, bool b_kc, bool a_vec, bool b_vec,
                       int batch, hipStream_t stream)
{
    constexpr int V = 16 / (int)sizeof(T);
    const int tiles = a.tiles;
    const dim3 grid((unsigned)(a.num_full + (tiles - a.num_full) * a.split), 1, (unsigned)batch);
    const dim3 block(256);
    const int sel = (a_kc ? 8 : 0) | (b_kc ? 4 : 0) | (a_vec ? 2 : 0) | (b_vec ? 1 : 0);
#define SBX_LAUNCH(AK, BKC, VA, VB) \
    gemm_mfma_kernel<T, BM, BN, BK, WM, WN, AK, BKC, VA, VB, PF, WPE><<<grid, block, 0, stream>>>(a)
    switch (sel) {
    case 0: SBX_LAUNCH(false, false, 1, 1); break;
    case 1: SBX_LAUNCH(false, false, 1, V); break;
    case 2: SBX_LAUNCH(false, false, V, 1); break;
    case 3: SBX_LAUNCH(false, false, V, V); break;
    case 4: SBX_LAUNCH(false, true, 1, 1); break;
    case 5: SBX_LAUNCH(false, true, 1, V); break;
    case 6: SBX_LAUNCH(false, true, V, 1); break;
    case 7: SBX_LAUNCH(false, true, V, V); break;
    case 8: SBX_LAUNCH(true, false, 1, 1); break;
    case 9: SBX_LAUNCH(true, false, 1, V); break;
    case 10: SBX_LAUNCH(true, false, V, 1); break;
    case 11: SBX_LAUNCH(true, false, V, V); break;
    case 12: SBX_LAUNCH(true, true, 1, 1); break;
    case 13: SBX_LAUNCH(true, true, 1, V); break;
    case 14: SBX_LAUNCH(true, true, V, 1); break;
    default: SBX_LAUNCH(true, true, V, V); break;
    }
#undef SBX_LAUNCH
    if (a.split > 1) {
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        constexpr int CHUNKS = BM * BN / 256;
        const dim3 rgrid((unsigned)((tiles - a.num_full) * CHUNKS), 1, (unsigned)batch);
        splitk_reduce_kernel<T, BM, BN><<<rgrid, block, 0, stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace sbx
