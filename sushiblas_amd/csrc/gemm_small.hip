// gemm_small.hip -- one-launch fp32 GEMM for small problems.
//
// The MFMA tile kernel (gemm_mfma.hpp) fills the 256 CUs of a small problem
// only by cutting K across workgroups, which costs a second kernel that sums
// the parts.  Here each workgroup owns one 32x32 tile of C (one
// v_mfma_f32_32x32x2_f32 block) and its four waves cut K four ways among
// themselves: every wave streams its k-range of A and B straight from
// global memory into MFMA operand registers (no LDS staging: the waves share
// no operand data), the four partial blocks meet in LDS once, and the sum --
// always wave 0 + 1 + 2 + 3, so the result is deterministic -- gets the
// alpha/beta (and ReLU) epilogue.  512^3 is 256 such tiles: one per CU.
//
// Operand registers follow the MFMA lane layout with the same k permutation
// as the tile kernel: inside a group of 8 k values, lane group q (= lane/32)
// at MFMA step kk uses k = 8g + 4q + kk.  A k-contiguous operand then feeds
// 4 steps from one 16-byte load per lane; an x-contiguous one needs a 4-byte
// load per step (32 lanes read 128 consecutive bytes of one row).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.hpp"

namespace sbx {
namespace {

constexpr int kStageGroups = 4;  // k groups of 8 per pipeline stage (32 k)

// One operand's registers for a stage of 32 k values: for group s and step
// kk, v[s][kk] is this lane's element (row/column i = lane % 32).
template <bool KC, bool KTAIL>
struct SmallOperand {
    float v[kStageGroups][4];

    // base: the operand at this stage's first k (k0) and the tile's first
    // row (KC: element (x, k) at x*ld + k; else (k, x) at k*ld + x).
    // k_lim: first k past this wave's range; k_end: K.
    __device__ inline void load(const float* base, int64_t span_bytes, int64_t ld, int i, int q,
                                bool x_ok, int k0, int k_lim, int k_end)
    {
        const __amdgpu_buffer_rsrc_t r = make_rsrc(base, span_bytes);
#pragma unroll
        for (int s = 0; s < kStageGroups; ++s) {
            const int kq = 8 * s + 4 * q;  // first k of this lane's quad, stage-relative
            if (KC) {
                const bool ok = x_ok && k0 + kq < k_lim;
                const int off = ok ? (int)(((int64_t)i * ld + kq) * 4) : kOobOffset;
                u32x4 w = raw_load16(r, off);
                if (KTAIL) {
                    // elements past K hold the next row's first values
                    const int lim = k_end - (k0 + kq);
#pragma unroll
                    for (int e = 1; e < 4; ++e) w[e] = e < lim ? w[e] : 0u;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) v[s][e] = __uint_as_float(w[e]);
            } else {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    // rows past the X extent only reach C entries never stored
                    const bool ok = k0 + kq + kk < k_lim;
                    const int off = ok ? (int)(((int64_t)(kq + kk) * ld + i) * 4) : kOobOffset;
                    v[s][kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
                }
            }
        }
    }
};

template <bool A_KC, bool B_KC, bool KTAIL>
__global__ void __launch_bounds__(256) gemm_small_kernel(GemmArgs<float> p)
{
    __shared__ float red[4 * 1024];  // the four waves' partial blocks
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int i = lane & 31, q = lane >> 5;
    const int tm = (int)(blockIdx.x % (unsigned)p.tiles_m);
    const int tn = (int)(blockIdx.x / (unsigned)p.tiles_m);
    const int m0 = tm * 32, n0 = tn * 32;
    const float* A;
    const float* B;
    float* C;
    batch_bases(p, (int64_t)blockIdx.z, A, B, C);

    // this wave's k groups [g0, g1) of the ceil(K/8); k past k_lim is zeroed
    const int ng = (p.K + 7) / 8;
    const int g0 = (int)((int64_t)wave * ng / 4);
    const int g1 = (int)((int64_t)(wave + 1) * ng / 4);
    const int k_lim = min(p.K, 8 * g1);
    const bool a_ok = m0 + i < p.M, b_ok = n0 + i < p.N;

    // operand origin (tile, k = 0) and the bytes from there to the matrix end
    const int64_t a_org = A_KC ? (int64_t)m0 * p.lda : (int64_t)m0;
    const int64_t b_org = B_KC ? (int64_t)n0 * p.ldb : (int64_t)n0;
    const int64_t a_end = A_KC ? (int64_t)(p.M - 1) * p.lda + p.K : (int64_t)(p.K - 1) * p.lda + p.M;
    const int64_t b_end = B_KC ? (int64_t)(p.N - 1) * p.ldb + p.K : (int64_t)(p.K - 1) * p.ldb + p.N;
    auto a_at = [&](int k0) { return a_org + (A_KC ? (int64_t)k0 : (int64_t)k0 * p.lda); };
    auto b_at = [&](int k0) { return b_org + (B_KC ? (int64_t)k0 : (int64_t)k0 * p.ldb); };

    SmallOperand<A_KC, KTAIL> a[2];
    SmallOperand<B_KC, KTAIL> b[2];
    auto issue = [&](int st, int k0) {
        const int64_t pa = a_at(k0), pb = b_at(k0);
        a[st].load(A + pa, (a_end - pa) * 4, p.lda, i, q, a_ok, k0, k_lim, p.K);
        b[st].load(B + pb, (b_end - pb) * 4, p.ldb, i, q, b_ok, k0, k_lim, p.K);
    };

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    auto mma = [&](int st) {
#pragma unroll
        for (int s = 0; s < kStageGroups; ++s)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[st].v[s][kk], b[st].v[s][kk], acc,
                                                           0, 0, 0);
    };

    // two stages in flight; loads past the range are masked to zero, so the
    // next stage is issued unconditionally (a wave with no k groups runs one
    // all-zero stage)
    const int ke = 8 * g1;
    int k0 = 8 * g0;
    issue(0, k0);
    for (;;) {
        issue(1, k0 + 32);
        mma(0);
        k0 += 32;
        if (k0 >= ke) break;
        issue(0, k0 + 32);
        mma(1);
        k0 += 32;
        if (k0 >= ke) break;
    }

    // partial blocks -> LDS, element (lane, r) at r * 64 + lane
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave * 1024 + r * 64 + lane] = acc[r];
    __syncthreads();

    // each lane finishes 4 elements of the 32x32 tile
    const float alpha = p.alpha, beta = p.beta;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = u * 256 + tid;
        const int el = e & 63, r = e >> 6;
        const float sum = ((red[e] + red[1024 + e]) + red[2048 + e]) + red[3072 + e];
        const int row = Mfma<float>::row(r, el >> 5), col = el & 31;
        const int m = m0 + row, n = n0 + col;
        if (m < p.M && n < p.N) {
            float* cp = C + (int64_t)m * p.ldc + n;
            float v = alpha * sum;
            if (beta != 0.0f) v += beta * *cp;
            *cp = p.relu ? relu_of(v) : v;
        }
    }
}

}  // namespace

hipError_t launch_small(const GemmArgs<float>& a, bool a_kc, bool b_kc, int batch,
                        hipStream_t stream)
{
    const dim3 grid((unsigned)(a.tiles_m * a.tiles_n), 1, (unsigned)batch);
    const dim3 block(256);
    const bool tail = (a_kc || b_kc) && a.K % 4 != 0;
#define SBX_LAUNCH(AK, BKC, TAIL) gemm_small_kernel<AK, BKC, TAIL><<<grid, block, 0, stream>>>(a)
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
    return hipGetLastError();
}

}  // namespace sbx
