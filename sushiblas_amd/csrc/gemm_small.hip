// gemm_small.hip -- one-launch GEMM for small problems (fp32 and fp64).
//
// The MFMA tile kernel (gemm_mfma.hpp) fills the 256 CUs of a small problem
// only by cutting K across workgroups, which costs a second kernel that sums
// the parts.  Here each workgroup owns one 32x32 tile of C and its NW = 4
// or 8 waves cut K NW ways among themselves: every wave streams its k-range
// of A and B straight from global memory into MFMA operand registers (no LDS
// staging: the waves share no operand data), the NW partial tiles meet in
// LDS once, and the sum -- always in wave order, so the result is
// deterministic -- gets the alpha/beta (and ReLU) epilogue.  512^3 is 256
// such tiles: one per CU.  fp32 runs one v_mfma_f32_32x32x2_f32 block per
// wave; fp64 a 2x2 grid of v_mfma_f64_16x16x4_f64 blocks.
//
// Operand registers follow the MFMA lane layout with the same k permutation
// as the tile kernel: inside a group of 8 k values, lane group q at MFMA step
// kk uses k = 8g + V*q + kk (V = 16 bytes / sizeof(T)).  A k-contiguous
// operand then feeds V steps from one 16-byte load per lane; an
// x-contiguous one needs one element load per step (the lanes of a group
// read consecutive elements of one row).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.hpp"

namespace sbx {
namespace {

constexpr int kTile = 32;        // workgroup tile edge
// k groups of 8 per pipeline stage, per form: 32 k for the 4-wave form, 16 k
// for the 8-wave one, whose waves each hold half as much K (timed in
// rotation at 512^2 x K, results bit-identical: the 8-wave form 5 % faster
// at K = 512 and 16 % at K = 2048 with 16-k stages; the 4-wave form no
// faster from K = 512 on, with 16 or with 64)
template <int NW>
constexpr int stage_groups()
{
    return NW == 8 ? 2 : 4;
}

// n / d for wave-uniform n < 2^22, d > 0: the float quotient through the
// hardware reciprocal (1 ulp) is within 1 of the integer one, and one
// correction each way makes it exact.  The integer division the compiler
// would emit takes about 40 scalar instructions, which every wave of a CU
// issues through the CU's one scalar unit before its first load.  The
// quotient is read back through readfirstlane so that the compiler keeps
// what is built from it (the buffer descriptors) in scalar registers.
__device__ inline unsigned udiv22(unsigned n, unsigned d)
{
    const unsigned q = (unsigned)__builtin_amdgcn_readfirstlane(
        (int)(unsigned)((float)n * __builtin_amdgcn_rcpf((float)d)));
    const int r = (int)(n - q * d);
    return q + (unsigned)(r >= (int)d) - (unsigned)(r < 0);
}

// One element of T from a raw buffer load (4 or 8 bytes).
__device__ inline float load_elem(float*, __amdgpu_buffer_rsrc_t r, int off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ inline double load_elem(double*, __amdgpu_buffer_rsrc_t r, int off)
{
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return __hiloint2double((int)w.y, (int)w.x);
}

// One operand's registers for a stage of SG groups of 8 k values: for block b (of NB
// along the operand's m or n), group s and step kk, v[b][s][kk] is this
// lane's element (row/column b*MB + lane % MB of the tile).
template <typename T, bool KC, bool KTAIL, int SG>
struct SmallOperand {
    typedef Mfma<T> MF;
    static constexpr int MB = MF::MB, V = MF::V, NB = kTile / MB;
    T v[NB][SG][V];

    // base: the operand at this stage's first k (k0) and the tile's first
    // row (KC: element (x, k) at x*ld + k; else (k, x) at k*ld + x).
    // x_rem: rows/columns of the tile inside the matrix; k_lim: first k past
    // this wave's range; k_end: K.
    __device__ inline void load(const T* base, int64_t span_bytes, int64_t ld, int i, int q,
                                int x_rem, int k0, int k_lim, int k_end, int only)
    {
        const __amdgpu_buffer_rsrc_t r = make_rsrc(base, span_bytes);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int x = b * MB + i;
#pragma unroll
            for (int s = 0; s < SG; ++s) {
                if (only >= 0 && s != only) continue;  // one group (a constant after inlining)
                const int kq = 8 * s + V * q;  // first k of this lane's run, stage-relative
                if (KC) {
                    const bool ok = x < x_rem && k0 + kq < k_lim;
                    const int off = ok ? (int)(((int64_t)x * ld + kq) * (int64_t)sizeof(T))
                                       : kOobOffset;
                    u32x4 w = raw_load16(r, off);
                    if (KTAIL) {
                        // elements past K hold the next row's first values
                        constexpr int DPE = (int)sizeof(T) / 4;
                        const int lim = k_end - (k0 + kq);
#pragma unroll
                        for (int d = DPE; d < 4; ++d) w[d] = d / DPE < lim ? w[d] : 0u;
                    }
                    if constexpr (sizeof(T) == 4) {
#pragma unroll
                        for (int e = 0; e < V; ++e) v[b][s][e] = __uint_as_float(w[e]);
                    } else {
#pragma unroll
                        for (int e = 0; e < V; ++e)
                            v[b][s][e] = __hiloint2double((int)w[2 * e + 1], (int)w[2 * e]);
                    }
                } else {
#pragma unroll
                    for (int kk = 0; kk < V; ++kk) {
                        // rows past the X extent only reach C entries never stored
                        const bool ok = k0 + kq + kk < k_lim;
                        const int off =
                            ok ? (int)(((int64_t)(kq + kk) * ld + x) * (int64_t)sizeof(T))
                               : kOobOffset;
                        v[b][s][kk] = load_elem((T*)nullptr, r, off);
                    }
                }
            }
        }
    }
};

// The arguments the first operand loads depend on come first, as separate
// scalars (14 dwords): this file is compiled with kernel-argument preloading,
// so the dispatcher places them in SGPRs before the first instruction and
// the loads go out without a trip to the argument buffer (a firmware without
// preloading runs a compiled-in prologue that loads them instead).  `group`
// is -1 for a strided launch, else the grouped launch's operand swap (0/1),
// whose device table comes from p.  Everything the epilogue needs -- C, its
// strides, the scalars -- is read from p after the k loop, so no wait for
// it stands before the operand loads.  BETA: beta != 0 (C is read); the
// beta = 0 form has no trace of the C loads, whose run-time test and index
// work slowed it by 1-6 % at short K.  ALT (8 waves only): the two waves
// sharing each SIMD take turns at the higher issue priority, stage by stage.
template <typename T, int NW, bool A_KC, bool B_KC, bool KTAIL, bool BETA, bool ALT>
__global__ void __launch_bounds__(NW * 64)
gemm_small_kernel(const T* A, const T* B, int lda, int ldb, int M, int N, int K, int group,
                  int64_t str_a, int64_t str_b, GemmArgs<T> p)
{
    typedef Mfma<T> MF;
    constexpr int MB = MF::MB, V = MF::V, NB = kTile / MB, NACC = MF::NACC;
    constexpr int PART = NB * NB * NACC * 64;  // one wave's partial tile
    static_assert(PART == kTile * kTile, "a wave's blocks cover the tile once");
    __shared__ T red[NW * PART];  // the waves' partial tiles
    probe_mark(p, 0);  // kernel entry

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // uniform per wave, and known to be: the buffer descriptors built from
    // it below stay scalar (as a vector value every load would need a loop
    // over the distinct descriptors of the wave)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane % MB, q = lane / MB;
    // grid (tiles_m, tiles_n, batch).  The hardware deals workgroups to the
    // 8 XCDs round-robin by linear index, each XCD with its own L2.  For a
    // long K, when an entry's tile count is a multiple of 8 (so that every
    // entry deals alike), the tiles are renumbered so that XCD j takes the
    // j-th eighth of them, walked in columns G tiles tall: an XCD then covers
    // about a sqrt(tiles / 8)-wide square, whose A and B panels its L2
    // shares, instead of every column of tiles (512^2 x 2048: 17.9 against
    // 21.2 us on the 4-wave form, 14.5 against 15.5 on the 8-wave one).
    // Below K = 1024 the renumbering's scalar work, done by every wave before
    // its first load, cost more than the L2 saved (512^3: first loads 0.2 us
    // later).
    int tm = (int)blockIdx.x, tn = (int)blockIdx.y;
    if (K >= 1024) {
        const unsigned gx = (unsigned)(M + kTile - 1) / kTile;  // gridDim.x
        const unsigned gy = (unsigned)(N + kTile - 1) / kTile;  // gridDim.y
        const unsigned tiles = gx * gy;
        if ((tiles & 7u) == 0 && tiles > 8 && tiles <= (1u << 22)) {
            const unsigned lin = (unsigned)tm + gx * (unsigned)tn;
            const unsigned eighth = tiles >> 3;
            const unsigned id = (lin & 7u) * eighth + (lin >> 3);
            const unsigned G = 1u << ((31 - __builtin_clz(eighth)) >> 1);  // ~sqrt(eighth)
            const unsigned span = G * gy;
            const unsigned grp = udiv22(id, span);
            const unsigned first = grp * G;
            const unsigned gs = min(gx - first, G);
            const unsigned in = id - grp * span;
            const unsigned col = udiv22(in, gs);
            tm = (int)(first + in - col * gs);
            tn = (int)col;
        }
    }
    const int m0 = tm * kTile, n0 = tn * kTile;
    const int64_t z = (int64_t)blockIdx.z;
    if (group >= 0) {  // grouped launch: entry z's operands from the device table
        const void* const* e = p.table + 3 * z;
        A = static_cast<const T*>(e[group ? 1 : 0]);
        B = static_cast<const T*>(e[group ? 0 : 1]);
    } else {
        A += z * str_a;
        B += z * str_b;
    }

    // this wave's k groups [g0, g1) of the ceil(K/8); k past k_lim is zeroed
    const int ng = (K + 7) / 8;
    const int g0 = (int)((int64_t)wave * ng / NW);
    const int g1 = (int)((int64_t)(wave + 1) * ng / NW);
    const int k_lim = min(K, 8 * g1);

    // operand origin (tile, k = 0) and the elements from there to the matrix end
    const int64_t a_org = A_KC ? (int64_t)m0 * lda : (int64_t)m0;
    const int64_t b_org = B_KC ? (int64_t)n0 * ldb : (int64_t)n0;
    const int64_t a_end = A_KC ? (int64_t)(M - 1) * lda + K : (int64_t)(K - 1) * lda + M;
    const int64_t b_end = B_KC ? (int64_t)(N - 1) * ldb + K : (int64_t)(K - 1) * ldb + N;
    auto a_at = [&](int k0) { return a_org + (A_KC ? (int64_t)k0 : (int64_t)k0 * lda); };
    auto b_at = [&](int k0) { return b_org + (B_KC ? (int64_t)k0 : (int64_t)k0 * ldb); };

    constexpr int SG = stage_groups<NW>();
    constexpr int kStageK = 8 * SG;  // k values per stage
    SmallOperand<T, A_KC, KTAIL, SG> a[2];
    SmallOperand<T, B_KC, KTAIL, SG> b[2];
    // The fp32 4-wave form's stages (4 groups) issue A's and B's loads group
    // by group, so that the first MFMAs wait only for their own group's data
    // (in-order load counters: 512^2 x 2048 17.7 -> 15.8 us, 512^3 6.2 ->
    // 6.15, bit-identical); the 8-wave form (2 groups) and fp64 issue all of
    // A then all of B, which measured faster there (512^3 5.5 against 5.9 us
    // on 8 waves; fp64 1024^2 x 512 27.4 against 29.1 us).
    auto issue = [&](int st, int k0) {
        const int64_t pa = a_at(k0), pb = b_at(k0);
        const int64_t sa = (a_end - pa) * (int64_t)sizeof(T), sb = (b_end - pb) * (int64_t)sizeof(T);
        if constexpr (NW == 4 && sizeof(T) == 4) {
#pragma unroll
            for (int s = 0; s < SG; ++s) {
                a[st].load(A + pa, sa, lda, i, q, M - m0, k0, k_lim, K, s);
                b[st].load(B + pb, sb, ldb, i, q, N - n0, k0, k_lim, K, s);
            }
        } else {
            a[st].load(A + pa, sa, lda, i, q, M - m0, k0, k_lim, K, -1);
            b[st].load(B + pb, sb, ldb, i, q, N - n0, k0, k_lim, K, -1);
        }
    };

    typename MF::acc_t acc[NB][NB];
#pragma unroll
    for (int bi = 0; bi < NB; ++bi)
#pragma unroll
        for (int bj = 0; bj < NB; ++bj)
#pragma unroll
            for (int r = 0; r < NACC; ++r) acc[bi][bj][r] = 0;
    auto mma = [&](int st) {
#pragma unroll
        for (int s = 0; s < SG; ++s)
#pragma unroll
            for (int kk = 0; kk < V; ++kk)
#pragma unroll
                for (int bi = 0; bi < NB; ++bi)
#pragma unroll
                    for (int bj = 0; bj < NB; ++bj)
                        acc[bi][bj] = MF::mma(a[st].v[bi][s][kk], b[st].v[bj][s][kk], acc[bi][bj]);
    };

    // n stages of kStageK k in two register sets (stage i in set i % 2).  Inside
    // the loop the next stage is issued unconditionally; the last one or two
    // stages are peeled so that nothing is loaded past the range (a load
    // whose result is never used still delays the epilogue, which reuses
    // its registers, by a full memory round trip).  The compiler places a
    // stage's loads among the previous stage's MFMAs once their registers
    // are free, so about one stage is in flight; pinning two (three register
    // sets, loads between scheduling barriers) measured slower.
    const int ke = 8 * g1;
    int k0 = 8 * g0;
    const int n = (ke - k0 + kStageK - 1) / kStageK;
    if (n > 0) issue(0, k0);
    probe_mark(p, 1);  // first stage's loads issued
    // With ALT the two waves sharing each SIMD (w and w + 4) take turns at
    // the higher issue priority, one stage each: under the default
    // oldest-first issue one runs ahead and the other finishes alone, its
    // loads no longer hidden behind its partner's MFMAs.  Each half of the
    // workgroup runs its own copy of the loop, so that no branch splits a
    // stage's loads from the MFMAs the compiler interleaves them with (a
    // run-time test there slowed the loop even with the turns off).
    auto run = [&](auto first) {
        constexpr bool F = decltype(first)::value;
        auto favour = [&](int stage) {
            if constexpr (ALT) {
                if constexpr (F) {
                    if (stage == 0) __builtin_amdgcn_s_setprio(1);
                    else __builtin_amdgcn_s_setprio(0);
                } else {
                    if (stage == 0) __builtin_amdgcn_s_setprio(0);
                    else __builtin_amdgcn_s_setprio(1);
                }
            }
        };
        int done = 0;  // stages consumed
        for (; done + 2 < n; done += 2) {
            issue(1, k0 + kStageK);
            favour(0);
            mma(0);
            issue(0, k0 + 2 * kStageK);
            favour(1);
            mma(1);
            k0 += 2 * kStageK;
        }
        if (n - done == 2) {
            issue(1, k0 + kStageK);
            favour(0);
            mma(0);
            favour(1);
            mma(1);
        } else if (n - done == 1) {
            mma(0);
        }
        if constexpr (ALT) __builtin_amdgcn_s_setprio(0);
    };
    if constexpr (ALT) {
        if ((wave >> 2) == 0) run(std::true_type{});
        else run(std::false_type{});
    } else {
        run(std::true_type{});
    }
    probe_mark(p, 2);  // this wave's MFMAs issued

    // each lane finishes PER = 1024 / (64 NW) elements of the 32x32 tile:
    // element e = u*64*NW + tid of the partial-tile layout below
    constexpr int PER = kTile * kTile / (NW * 64);
    auto c_index = [&](int u, int& m, int& n) {
        const int e = u * (NW * 64) + tid;
        const int el = e & 63, r = (e >> 6) % NACC, blk = (e >> 6) / NACC;
        m = m0 + (blk / NB) * MB + MF::row(r, el / MB);
        n = n0 + (blk % NB) * MB + el % MB;
    };
    typedef __attribute__((address_space(1))) T GlobalT;
    auto c_base = [&]() {
        T* C = group >= 0 ? static_cast<T*>(const_cast<void*>(p.table[3 * z + 2]))
                          : p.C + z * p.str_c;
        return (GlobalT*)C;
    };

    // partial tiles -> LDS, element (bi, bj, r, lane) at ((bi*NB + bj)*NACC + r)*64 + lane
#pragma unroll
    for (int bi = 0; bi < NB; ++bi)
#pragma unroll
        for (int bj = 0; bj < NB; ++bj)
#pragma unroll
            for (int r = 0; r < NACC; ++r)
                red[wave * PART + ((bi * NB + bj) * NACC + r) * 64 + lane] = acc[bi][bj][r];

    // With beta != 0 this lane's old C values are loaded now, between the
    // partial tiles' writes and the barrier, so that their latency overlaps
    // the wait for the slowest wave (loaded after the barrier, each was a
    // dependent round trip to memory: 37x1000x300, 4 waves, 6.4 -> 5.5 us).
    // The details matter to the compiler:
    //  * after the writes, whose accumulators are then dead (a branch while
    //    they lived made it copy all of them);
    //  * a lane whose element lies outside C reads the tile's first element
    //    (in C) and discards it (masked loads merged with a default made it
    //    wait for the first load before issuing the next);
    //  * a global-address-space pointer (a flat load would also count in the
    //    LDS writes' wait before the barrier, which would then wait for C).
    // Without BETA, C's address is formed after the barrier, as the stores
    // need it (formed before it, fp64 256^3 ran 3 % slower).
    GlobalT* Cg = nullptr;
    [[maybe_unused]] T c_old[PER];  // BETA only
    if constexpr (BETA) {
        Cg = c_base();
        const int64_t ldc = p.ldc;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            int m, n;
            c_index(u, m, n);
            const bool in = m < M && n < N;
            c_old[u] = Cg[in ? (int64_t)m * ldc + n : (int64_t)m0 * ldc + n0];
        }
    }

    __syncthreads();

    // the waves' partials summed in wave order
    if constexpr (!BETA) Cg = c_base();
    const int64_t ldc = p.ldc;
    const T alpha = p.alpha;
    const int relu = p.relu;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int e = u * (NW * 64) + tid;
        T sum = red[e];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += red[w * PART + e];
        int m, n;
        c_index(u, m, n);
        if (m < M && n < N) {
            T v = alpha * sum;
            if constexpr (BETA) v += p.beta * c_old[u];
            Cg[(int64_t)m * ldc + n] = relu ? relu_of(v) : v;
        }
    }
    probe_mark(p, 3);  // C stores issued
}

}  // namespace

namespace {
template <typename T, int NW, bool A_KC, bool B_KC, bool KTAIL, bool BETA>
void launch_one(dim3 grid, dim3 block, hipStream_t stream, const GemmArgs<T>& a)
{
    const int group = a.table ? a.table_swap : -1;
    if constexpr (NW == 8) {
        if (a.alt_prio) {
            gemm_small_kernel<T, NW, A_KC, B_KC, KTAIL, BETA, true><<<grid, block, 0, stream>>>(
                a.A, a.B, (int)a.lda, (int)a.ldb, a.M, a.N, a.K, group, a.str_a, a.str_b, a);
            return;
        }
    }
    gemm_small_kernel<T, NW, A_KC, B_KC, KTAIL, BETA, false><<<grid, block, 0, stream>>>(
        a.A, a.B, (int)a.lda, (int)a.ldb, a.M, a.N, a.K, group, a.str_a, a.str_b, a);
}

template <typename T, int NW>
hipError_t launch_small_nw(const GemmArgs<T>& a, bool a_kc, bool b_kc, int batch,
                           hipStream_t stream)
{
    const dim3 grid((unsigned)a.tiles_m, (unsigned)a.tiles_n, (unsigned)batch);
    const dim3 block(NW * 64);
    // leading dimensions go in as 32-bit scalars (the planner's offset check
    // keeps a 32-row tile's offsets, so ld itself, far below 2^31)
    if (a.lda > INT32_MAX || a.ldb > INT32_MAX) return hipErrorInvalidValue;
    const bool tail = (a_kc || b_kc) && a.K % (16 / (int)sizeof(T)) != 0;
    const bool beta = a.beta != (T)0;
#define SBX_LAUNCH(AK, BKC, TAIL)                                                  \
    (beta ? launch_one<T, NW, AK, BKC, TAIL, true>(grid, block, stream, a)         \
          : launch_one<T, NW, AK, BKC, TAIL, false>(grid, block, stream, a))
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
}  // namespace

template <typename T>
hipError_t launch_small(const GemmArgs<T>& a, bool a_kc, bool b_kc, int batch, hipStream_t stream,
                        int waves)
{
    if (waves == 4) return launch_small_nw<T, 4>(a, a_kc, b_kc, batch, stream);
    // 8 waves: fp32 only (the planner offers no fp64 form of it)
    if constexpr (sizeof(T) == 4) {
        if (waves == 8) return launch_small_nw<T, 8>(a, a_kc, b_kc, batch, stream);
    }
    return hipErrorInvalidValue;
}

template hipError_t launch_small<float>(const GemmArgs<float>&, bool, bool, int, hipStream_t, int);
template hipError_t launch_small<double>(const GemmArgs<double>&, bool, bool, int, hipStream_t,
                                         int);

}  // namespace sbx
