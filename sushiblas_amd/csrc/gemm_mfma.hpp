// gemm_mfma.hpp -- gfx950 (CDNA4) MFMA GEMM kernel template for fp32 and fp64.
//
// Computes, for row-major storage (column-major calls are mapped onto this by
// the dispatcher with C^T = op(B)^T op(A)^T):
//     C[m][n] = alpha * sum_k op(A)[m][k] * op(B)[k][n] + beta * C[m][n]
// which is the arithmetic the reference hands to oneMKL's
// row_major::gemm / gemm_batch (src/ops/blas/level3/gemm.cpp:58,63).
//
// Design (one workgroup = WAVES_M x WAVES_N wave64s -- 4, or 8 for the
// largest fp32 tile -- and one macro tile BM x BN):
//  * Operands go global -> VGPR staging -> LDS -> VGPR fragments -> MFMA.
//    Each operand keeps in LDS the layout it has in global memory, so every
//    global read is a coalesced 16-byte buffer load along the contiguous
//    dimension and every LDS write is a straight vector store (no transposing
//    scatter):
//      "k-contiguous"  tile (A not transposed / B transposed): [X][BK + PAD]
//      "x-contiguous"  tile (A transposed / B not transposed): [BK][X]
//  * Fragments are read with one 16-byte LDS read per lane.  The MFMA k index
//    is a permutation of the real k inside each k group of KG = Q*V values
//    (8; 16 for the 16x16x4 fp32 shape): lane group q at MFMA step kk uses
//    k = KG*g + V*q + kk (V = 16 bytes / sizeof(T)).  For an
//    x-contiguous tile, U neighbouring MFMA blocks are interleaved (block u
//    owns rows U*i + u) so that one 16-byte read feeds U blocks.
//  * Masking: loads go through buffer resources whose base moves with the
//    k tile; a vector that starts outside [0,M)x[0,K) (or [0,K)x[0,N)) gets
//    the offset 0x80000000, which the buffer unit turns into zeros.  The k
//    tiles that are full and not the last skip that per-step work: one
//    descriptor per operand fixed at the tile's k = 0 origin, a scalar
//    offset for the k tile, and only the (per-tile) X test.  Every
//    load is 16 bytes, also for odd leading dimensions (4/8-byte aligned
//    addresses); a k-contiguous vector that straddles K is zeroed past K
//    before its LDS write.  Ragged M/N/K and unaligned leading dimensions
//    need no separate kernel.
//  * LDS is double-buffered: the global loads for tile t+1 are issued before
//    the MFMAs of tile t, stored to the other LDS buffer after them, and one
//    barrier per k-tile separates producer and consumer.
//  * The 1-D grid is remapped so that consecutive tiles land on the same XCD
//    (hardware deals workgroups round-robin over the 8 XCDs) and, inside an
//    XCD, walk a GROUP_M-tall column of tiles so that A row-panels and B
//    column-panels are shared through that XCD's L2.
//  * SYRK (src/ops/blas/level3/syrk.cpp:84-194) runs through the same kernel
//    with B = A and `uplo` set: only the tiles that meet the requested
//    triangle are enumerated, and diagonal tiles store only the triangle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace sbx {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// MFMA shapes.  fp32: v_mfma_f32_32x32x2_f32 (MI = 0) or
// v_mfma_f32_16x16x4_f32 (MI = 1); fp64: v_mfma_f64_16x16x4_f64.
//   A operand: lane l holds A[i = l % MB][k = l / MB]
//   B operand: lane l holds B[k = l / MB][j = l % MB]
//   D: lane l, accumulator r holds D[row(r, l / MB)][l % MB]
//   (all layouts were confirmed on the device with one-hot probes)
// A k group is Q * V consecutive k values: one V-wide fragment read per
// lane feeds V MFMA steps.
// ---------------------------------------------------------------------------
template <typename T, int MI = 0>
struct Mfma;

template <>
struct Mfma<float, 0> {
    static constexpr int MB = 32;    // output block edge
    static constexpr int Q = 2;      // lane groups along k (= MFMA k)
    static constexpr int V = 4;      // elements per 16-byte read
    static constexpr int NACC = 16;  // accumulators per lane
    typedef f32x16 acc_t;
    __device__ static inline acc_t mma(float a, float b, acc_t c)
    {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    __device__ static inline int row(int r, int q) { return 8 * (r >> 2) + 4 * q + (r & 3); }
};

template <>
struct Mfma<float, 1> {
    static constexpr int MB = 16;
    static constexpr int Q = 4;
    static constexpr int V = 4;
    static constexpr int NACC = 4;
    typedef f32x4 acc_t;
    __device__ static inline acc_t mma(float a, float b, acc_t c)
    {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    __device__ static inline int row(int r, int q) { return 4 * q + r; }
};

template <>
struct Mfma<double, 0> {
    static constexpr int MB = 16;
    static constexpr int Q = 4;
    static constexpr int V = 2;
    static constexpr int NACC = 4;
    typedef f64x4 acc_t;
    __device__ static inline acc_t mma(double a, double b, acc_t c)
    {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
    }
    // measured on gfx950 with one-hot operands: row i sits in lane group i % 4,
    // accumulator i / 4 (unlike the fp32 16x16x4 form)
    __device__ static inline int row(int r, int q) { return q + 4 * r; }
};

// Cache-policy operand of a buffer load with the non-temporal (nt) bit set:
// the lines it brings in are the first to be evicted, for data read once.
constexpr int kNonTemporal = 2;

// Raw 16-byte buffer load.  The byte offset need only be 4-byte aligned:
// gfx950 serves unaligned multi-dword buffer loads (the device runs in
// unaligned access mode), and range-checks each dword on its own, so a load
// that straddles the end of the resource returns its in-range dwords and
// zeros for the rest (both checked on the device with in-bounds probes).
__device__ inline u32x4 raw_load16(__amdgpu_buffer_rsrc_t r, int off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Typed N-element LDS vector read (N * sizeof(T) in {4, 8, 16}).
template <typename T, int N>
struct LdsVec;
template <>
struct LdsVec<float, 1> {
    __device__ static inline void read(const float* p, float* o) { o[0] = *p; }
};
template <>
struct LdsVec<float, 2> {
    __device__ static inline void read(const float* p, float* o)
    {
        f32x2 v = *reinterpret_cast<const f32x2*>(p);
        o[0] = v.x; o[1] = v.y;
    }
};
template <>
struct LdsVec<float, 4> {
    __device__ static inline void read(const float* p, float* o)
    {
        f32x4 v = *reinterpret_cast<const f32x4*>(p);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
};
template <>
struct LdsVec<float, 3> {  // 12-byte aligned at best: element reads
    __device__ static inline void read(const float* p, float* o)
    {
        o[0] = p[0]; o[1] = p[1]; o[2] = p[2];
    }
};
template <>
struct LdsVec<double, 1> {
    __device__ static inline void read(const double* p, double* o) { o[0] = *p; }
};
template <>
struct LdsVec<double, 2> {
    __device__ static inline void read(const double* p, double* o)
    {
        f64x2 v = *reinterpret_cast<const f64x2*>(p);
        o[0] = v.x; o[1] = v.y;
    }
};

// Buffer resource word 3 for gfx9-family raw buffers (32-bit dword format).
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kOobOffset = static_cast<int>(0x80000000u);
constexpr int64_t kMaxRecords = 0x7ffffff0;

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes)
{
    int64_t n = bytes < 0 ? 0 : (bytes > kMaxRecords ? kMaxRecords : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n,
                                             kRsrcWord3);
}

template <typename T>
struct GemmArgs {
    const T* A;
    const T* B;
    T* C;
    int64_t lda, ldb, ldc;
    int64_t str_a, str_b, str_c;  // batch strides in elements (grid z)
    int M, N, K;
    T alpha, beta;
    int tiles_m, tiles_n;
    int group_m;
    bool c_vec;  // C rows allow 16-byte vector access (ldc, base and batch stride aligned)
    // Split-K of the tail: tiles [0, num_full) run whole; each tile in
    // [num_full, tiles_m*tiles_n) is cut into `split` k-ranges whose fp
    // partials go to ws (BM*BN elements per part), and splitk_reduce_kernel
    // sums them in part order and writes C.  split == 1: no split.
    int num_full;
    int split;
    T* ws;
    int relu;  // 1: C = max(alpha*A*B + beta*C, 0) with NaN -> 0 (fused ReLU epilogue)
    // Triangle-only output (SYRK): 0 = whole C; 1 = lower (column <= row);
    // 2 = upper (column >= row).  With uplo != 0, BM == BN, tiles_m ==
    // tiles_n = T and only the T(T+1)/2 tiles that meet the triangle exist.
    int uplo;
    int tiles;  // tiles in the grid: tiles_m * tiles_n, or T(T+1)/2 for a triangle
    // Grouped launch: batch entry z takes its operands from a device table of
    // 3 pointers per entry (A, B, C as the caller names them; with
    // table_swap the first two trade places, for the column-major mapping)
    // instead of base + z * stride.  Null: strided.
    const void* const* table;
    int table_swap;
    // Host side only: which operand the launch loads non-temporally (0
    // none, 1 A, 2 B), picking the kernel's STREAM variant.
    int stream_op;
    // Host side only, small-problem kernel's 8-wave form: run the variant
    // whose two waves sharing each SIMD take turns at the higher issue
    // priority (set for one-round grids with K >= 1024).
    int alt_prio;
#ifdef SBX_PROBE
    // Probe build only: per-workgroup timestamps of this dispatch (see
    // ProbeClock), for workgroups [0, stamp_blocks) of batch entry 0.
    unsigned long long* stamps;
    int stamp_blocks;
#endif
};

// ---------------------------------------------------------------------------
// Probe build (lib/libsbx_probe.so, compiled with SBX_PROBE; the product
// library has none of this): wave 0 of a workgroup reads the shader clock
// counter (s_memtime, core cycles) and the constant-rate real-time counter
// (s_memrealtime) at up to kStampPoints points of the kernel and stores each
// pair at once (nothing stays live across the k loop), so that the host can
// derive the clock and the busy cycles of every dispatch of a back-to-back
// timed loop without serialising it (counter collection by a profiler runs
// dispatches one at a time).
// ---------------------------------------------------------------------------
constexpr int kStampPoints = 4;

template <typename T>
__device__ inline void probe_mark(const GemmArgs<T>& p, int point)
{
#ifdef SBX_PROBE
    // A branch on a wave-uniform condition (wave 0, read into a scalar
    // register): on a per-lane one the compiler treats the kernel's later
    // values as divergent and builds its buffer descriptors in VGPRs.  Every
    // lane of wave 0 then stores the same 16 bytes.
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    // workgroup index within batch entry 0 (the small-problem kernel's grid is 2-D)
    const unsigned wg = blockIdx.x + blockIdx.y * gridDim.x;
    if (!p.stamps || wave != 0 || blockIdx.z != 0 || wg >= (unsigned)p.stamp_blocks) return;
    unsigned long long* d = p.stamps + ((size_t)wg * kStampPoints + point) * 2;
    const unsigned long long c = __builtin_amdgcn_s_memtime();
    const unsigned long long r = __builtin_amdgcn_s_memrealtime();
    d[0] = c;
    d[1] = r;
#else
    (void)p;
    (void)point;
#endif
}

// Operand and result bases of batch entry z.
template <typename T>
__device__ inline void batch_bases(const GemmArgs<T>& p, int64_t z, const T*& A, const T*& B, T*& C)
{
    if (p.table) {
        const void* const* e = p.table + 3 * z;
        A = static_cast<const T*>(e[p.table_swap ? 1 : 0]);
        B = static_cast<const T*>(e[p.table_swap ? 0 : 1]);
        C = static_cast<T*>(const_cast<void*>(e[2]));
    } else {
        A = p.A + z * p.str_a;
        B = p.B + z * p.str_b;
        C = p.C + z * p.str_c;
    }
}

// Tile id -> (tile row, tile column).
//  Whole C: GROUP_M-tall column walk, so consecutive ids share B column panels
//  and a group's A row panels.
//  Triangle (lower; upper is its mirror): the tile rows form bands of GROUP_M;
//  band [r0, r1) holds ids [r0(r0+1)/2, r1(r1+1)/2) and walks its columns in
//  order, top to bottom -- first the full-height columns left of the band's
//  diagonal block, then the triangular columns inside it -- the same panel
//  sharing as the GROUP_M walk, restricted to the triangle.
__device__ inline int64_t tri_count(int r) { return (int64_t)r * (r + 1) / 2; }

template <typename T>
__device__ inline void tile_coords(const GemmArgs<T>& p, int id, int& tm, int& tn)
{
    const int G = p.group_m;
    if (p.uplo == 0) {
        const int group_span = G * p.tiles_n;
        const int group = id / group_span;
        const int first_m = group * G;
        const int gsize = min(p.tiles_m - first_m, G);
        const int in_group = id - group * group_span;
        tm = first_m + in_group % gsize;
        tn = in_group / gsize;
        return;
    }
    // band of id: the plain row-by-row row index, rounded down to the band
    int r0 = (int)((sqrtf(8.0f * (float)id + 1.0f) - 1.0f) * 0.5f);
    r0 -= r0 % G;
    while (r0 > 0 && tri_count(r0) > id) r0 -= G;
    while (tri_count(min(r0 + G, p.tiles_m)) <= id) r0 += G;
    const int h = min(r0 + G, p.tiles_m) - r0;
    int rest = id - (int)tri_count(r0);
    int r, c;
    if (rest < r0 * h) {
        c = rest / h;
        r = r0 + rest % h;
    } else {
        rest -= r0 * h;
        int j = 0;  // column r0 + j of the diagonal block holds h - j tiles
        while (rest >= h - j) {
            rest -= h - j;
            ++j;
        }
        c = r0 + j;
        r = r0 + j + rest;
    }
    if (p.uplo == 1) { tm = r; tn = c; }
    else { tm = c; tn = r; }
}

// The reference's ReLU: x > 0 ? x : 0 (NaN and -0 become +0).
template <typename T>
__device__ inline T relu_of(T x)
{
    return x > (T)0 ? x : (T)0;
}

// ---------------------------------------------------------------------------
// One operand's global -> LDS pipeline, in 16-byte vectors (VEC elements)
// whatever the alignment of the leading dimension and base.
//   KC: the operand's k index is contiguous in memory (tile [X][BK+PAD]).
//   X : tile extent along m (for A) or n (for B).
//   KTAIL: K is not a multiple of VEC, so a k-contiguous vector may straddle K.
//   CPOL: cache-policy bits of the buffer loads (kNonTemporal or 0).
// ---------------------------------------------------------------------------
template <typename T, int X, int BK, bool KC, int PF, bool KTAIL, int NTHR = 256, int CPOL = 0>
struct Operand {
    static constexpr int V = 16 / (int)sizeof(T);
    static constexpr int VEC = V;  // elements per global load
    static constexpr int PAD = KC ? V : 0;
    static constexpr int LD = KC ? BK + PAD : X + PAD;          // LDS row pitch (elements)
    static constexpr int ELEMS = KC ? X * LD : BK * LD;         // LDS tile size (elements)
    static constexpr int CONTIG = KC ? BK : X;                   // contiguous extent of tile
    static constexpr int VPR = CONTIG / VEC;                     // vectors per tile row
    static constexpr int NV = X * BK / (VEC * NTHR);             // vectors per thread
    static_assert(X * BK % (VEC * NTHR) == 0, "tile not divisible over the lanes");
    typedef u32x4 raw_t;

    // Vector j of this thread is v = j*NTHR + tid of the tile, row
    // r = j*RSTEP + r0, column c0 (NTHR is a multiple of VPR, so the column
    // does not depend on j): only the j = 0 values are kept, the rest are
    // affine in j (fewer live registers than one entry per vector).
    static_assert(NTHR % VPR == 0, "rows per sweep must be whole");
    static constexpr int RSTEP = NTHR / VPR;  // tile rows covered per j
    int off0;          // byte offset of vector 0 relative to the tile base
    int off_step;      // byte offset between vectors j and j + 1 (RSTEP rows)
    int lds0;          // element offset of vector 0 in the LDS tile
    int r0, c0;        // tile row and column of vector 0
    int x_rem;         // rows/columns of the tile inside the matrix
    raw_t stage[PF][NV];  // register staging, PF tiles in flight
    int krem[PF];      // k extent left at the staged tile (k-tail masking)

    __device__ inline void init(int tid, int64_t ld, int x_rem_)
    {
        r0 = tid / VPR;
        c0 = (tid % VPR) * VEC;
        off0 = (int)((int64_t)r0 * ld + c0) * (int)sizeof(T);
        off_step = (int)((int64_t)RSTEP * ld) * (int)sizeof(T);
        lds0 = r0 * LD + c0;
        x_rem = x_rem_;
    }
    // k index of vector j within the tile and whether its X index is inside
    __device__ inline int kidx(int j) const { return KC ? c0 : r0 + j * RSTEP; }
    __device__ inline bool xok(int j) const { return KC ? r0 + j * RSTEP < x_rem : c0 < x_rem; }

    // A full k tile that is not the last (every vector inside K): the
    // descriptor stays at the tile's k = 0 origin and `soff` (scalar) moves
    // it to this k tile; only the X test remains, and it is the same for
    // every k tile.
    template <int S>
    __device__ inline void load_fixed(__amdgpu_buffer_rsrc_t rs, int soff, int k_rem)
    {
#pragma unroll
        for (int j = 0; j < NV; ++j)
            stage[S][j] = __builtin_amdgcn_raw_buffer_load_b128(
                rs, xok(j) ? off0 + j * off_step : kOobOffset, soff, CPOL);
        krem[S] = k_rem;
    }

    template <int S>
    __device__ inline void load(__amdgpu_buffer_rsrc_t rs, int k_rem)
    {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            bool ok = xok(j) && kidx(j) < k_rem;
            stage[S][j] = __builtin_amdgcn_raw_buffer_load_b128(
                rs, ok ? off0 + j * off_step : kOobOffset, 0, CPOL);
        }
        krem[S] = k_rem;
    }

    // A k-contiguous vector that straddles K holds, past K, the first
    // elements of the next row (or zeros past the buffer's end: the range
    // check is per dword): zero them.  An x-contiguous vector that straddles
    // the X extent needs nothing -- those elements only reach C rows/columns
    // that are never stored -- and its k index is one row, checked at load.
    // MASK: apply the k-tail zeroing (only the last k tile of K can hold a
    // straddling vector, so the k loop stores unmasked and only its peeled
    // tail masks)
    template <int S, bool MASK = true>
    __device__ inline void store(T* lds)
    {
        constexpr int DPE = (int)sizeof(T) / 4;  // dwords per element
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            raw_t w = stage[S][j];
            if constexpr (KC && KTAIL && MASK) {
                const int lim = krem[S] - kidx(j);  // elements of vector j inside K
#pragma unroll
                for (int d = DPE; d < VEC * DPE; ++d)
                    w[d] = d / DPE < lim ? w[d] : 0u;
            }
            *reinterpret_cast<raw_t*>(lds + lds0 + j * RSTEP * LD) = w;
        }
    }
};

// Fragment reader for one operand of one wave: NB blocks of MB along X.
template <typename T, int NB, bool KC, int LD, int MI = 0>
struct Frag {
    static constexpr int MB = Mfma<T, MI>::MB;
    static constexpr int V = Mfma<T, MI>::V;
    static constexpr int KG = Mfma<T, MI>::Q * V;  // k values per group
    static constexpr int U = KC ? 1 : (NB < V ? NB : V);  // interleave factor
    static_assert(NB % U == 0, "block count must be a multiple of the interleave");
    // LDS read instructions per k group: a k-contiguous tile takes one
    // 16-byte read per block; an x-contiguous one NB/U*V reads of U elements,
    // which the compiler pairs into ds_read2 instructions when they are
    // narrower than 16 bytes (rows kk and kk+1 lie LD elements apart), and
    // U = 3 (12 bytes at 4-byte alignment) takes two instructions each
    // (counted as one, the hint pattern missed most of them and the 48-column
    // tile ran 343 against 221 us at 65536 x 48 x 4096)
    static constexpr int INSTR = KC       ? NB
                                 : U == 3 ? (NB / U * V) * 2
                                          : (NB / U * V) / (U * (int)sizeof(T) < 16 ? 2 : 1);

    // Read the fragments of k-group g (KG k values) for wave offset w0.
    // f[b][kk] is block b's operand for MFMA step kk.
    __device__ static inline void read(const T* lds, int w0, int g, int lane, T (&f)[NB][V])
    {
        const int i = lane % MB, q = lane / MB;
        if (KC) {
#pragma unroll
            for (int b = 0; b < NB; ++b)
                LdsVec<T, V>::read(lds + (w0 + b * MB + i) * LD + g * KG + q * V, f[b]);
        } else {
#pragma unroll
            for (int s = 0; s < NB / U; ++s)
#pragma unroll
                for (int kk = 0; kk < V; ++kk) {
                    T t[U];
                    LdsVec<T, U>::read(lds + (g * KG + q * V + kk) * LD + w0 + s * U * MB + U * i, t);
#pragma unroll
                    for (int u = 0; u < U; ++u) f[s * U + u][kk] = t[u];
                }
        }
    }

    // X index (inside the wave tile) of row/column i of block b.
    __device__ static inline int map(int b, int i)
    {
        return KC ? b * MB + i : (b / U) * U * MB + U * i + (b % U);
    }
};

// Global-address-space pointer to T: epilogue loads and stores through it
// compile to global_* instructions (flat ones also count on lgkmcnt).
template <typename T>
struct Glob {
    typedef __attribute__((address_space(1))) T type;
};

// Typed vector store/load of U consecutive C elements (16 bytes for fp32 U=4).
// U consecutive elements of C one at a time: rows whose address or pitch
// does not allow vector access.
template <typename T, int U>
struct CElems {
    template <typename P>
    __device__ static inline void load(const P* p, T* o)
    {
#pragma unroll
        for (int u = 0; u < U; ++u) o[u] = p[u];
    }
    template <typename P>
    __device__ static inline void store(P* p, const T* v)
    {
#pragma unroll
        for (int u = 0; u < U; ++u) p[u] = v[u];
    }
};

template <typename T, int U>
struct CVec {
    template <typename P>
    __device__ static inline void load(const P* p, T* o)
    {
#pragma unroll
        for (int u = 0; u < U; ++u) o[u] = p[u];
    }
    template <typename P>
    __device__ static inline void store(P* p, const T* v)
    {
#pragma unroll
        for (int u = 0; u < U; ++u) p[u] = v[u];
    }
};
template <>
struct CVec<float, 4> {
    typedef Glob<f32x4>::type gv;
    __device__ static inline void load(const Glob<float>::type* p, float* o)
    {
        f32x4 v = *reinterpret_cast<const gv*>(p);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    __device__ static inline void store(Glob<float>::type* p, const float* v)
    {
        f32x4 w = {v[0], v[1], v[2], v[3]};
        *reinterpret_cast<gv*>(p) = w;
    }
};
template <>
struct CVec<float, 2> {
    typedef Glob<f32x2>::type gv;
    __device__ static inline void load(const Glob<float>::type* p, float* o)
    {
        f32x2 v = *reinterpret_cast<const gv*>(p);
        o[0] = v.x; o[1] = v.y;
    }
    __device__ static inline void store(Glob<float>::type* p, const float* v)
    {
        f32x2 w = {v[0], v[1]};
        *reinterpret_cast<gv*>(p) = w;
    }
};
template <>
struct CVec<double, 2> {
    typedef Glob<f64x2>::type gv;
    __device__ static inline void load(const Glob<double>::type* p, double* o)
    {
        f64x2 v = *reinterpret_cast<const gv*>(p);
        o[0] = v.x; o[1] = v.y;
    }
    __device__ static inline void store(Glob<double>::type* p, const double* v)
    {
        f64x2 w = {v[0], v[1]};
        *reinterpret_cast<gv*>(p) = w;
    }
};

template <int N>
using Int = std::integral_constant<int, N>;

// Slice x of n items cut into `slots` near-equal slices, in order.
__host__ __device__ constexpr int slice(int x, int n, int slots)
{
    return (x + 1) * n / slots - x * n / slots;
}
__host__ __device__ constexpr bool slices_cover(int n, int slots)
{
    int sum = 0;
    for (int x = 0; x < slots; ++x) {
        if (slice(x, n, slots) < 0) return false;
        sum += slice(x, n, slots);
    }
    return sum == n;
}
// the regions of the compiled tiles: more MFMAs than memory instructions,
// fewer, and equal
static_assert(slices_cover(96, 34) && slices_cover(16, 18) && slices_cover(32, 16) &&
                  slices_cover(5, 6) && slices_cover(0, 3),
              "hint slices must add up to the region's MFMAs");

// Scheduling hints for one region of a k step (see gemm_mfma_kernel's
// step).  hints_a: NLD global loads, NRD fragment reads, then MEM - NLD -
// NRD LDS writes, each followed by its slice of the region's MF MFMAs.
// hints_b: NRD fragment reads, each followed by its slice.  The slices add
// up to exactly the region's MFMAs: s_barrier does not bound MFMAs for the
// scheduler, so a group that asks for more takes them from the next region
// and pushes that region's memory instructions to its end.
template <int I, int NLD, int NRD, int MEM, int MF>
__device__ inline void hints_a()
{
    if constexpr (I < MEM) {
        constexpr int kind = I < NLD ? 0x020 : (I < NLD + NRD ? 0x100 : 0x200);
        __builtin_amdgcn_sched_group_barrier(kind, 1, 0);  // VMEM read / DS read / DS write
        constexpr int n = slice(I, MF, MEM);
        if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x008, n, 0);  // MFMA
        hints_a<I + 1, NLD, NRD, MEM, MF>();
    }
}
template <int I, int NRD, int MF>
__device__ inline void hints_b()
{
    if constexpr (I < NRD) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        constexpr int n = slice(I, MF, NRD);
        if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x008, n, 0);
        hints_b<I + 1, NRD, MF>();
    }
}

// PF: global tiles in flight (1 = the next tile is fetched while the current
// one is multiplied; 2 = the one after that too, for HBM-bound shapes).
// WPE: waves per SIMD the register budget is sized for (1 or 2).
// MI: MFMA shape (see Mfma; fp32 only has a choice).
// STREAM: the operand whose loads are non-temporal (0 none, 1 A, 2 B).
// BNC: columns of the tile that are computed (default BN).  BNC < BN loads a
// BN-wide B tile but runs MFMAs and keeps accumulators for its first BNC
// columns only: the host uses it where N <= BNC (one tile column), so a
// 48-wide C does not pay for 64 columns of MFMAs.  BMC: the same for rows.
template <typename T, int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool A_KC, bool B_KC,
          bool KTAIL, int PF, int WPE, int MI = 0, int STREAM = 0, int BNC = BN, int BMC = BM>
__global__ void __launch_bounds__(WAVES_M * WAVES_N * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_mfma_kernel(GemmArgs<T> p)
{
    typedef Mfma<T, MI> MF;
    constexpr int MB = MF::MB;
    constexpr int V = MF::V;
    constexpr int KG = MF::Q * V;  // k values per group
    constexpr int WTM = BMC / WAVES_M, WTN = BNC / WAVES_N;
    constexpr int NBM = WTM / MB, NBN = WTN / MB;
    static_assert(BNC <= BN && BNC % (WAVES_N * MB) == 0, "computed columns: whole blocks of BN");
    static_assert(BMC <= BM && BMC % (WAVES_M * MB) == 0, "computed rows: whole blocks of BM");
    constexpr int G = BK / KG;  // k groups per tile
    constexpr int NTHR = WAVES_M * WAVES_N * 64;
    static_assert(NTHR == 256 || NTHR == 512, "4 or 8 waves per workgroup");
    static_assert(BK % KG == 0, "BK must be a multiple of the k group");
    static_assert(PF >= 1 && PF <= 4, "prefetch depth 1 to 4");
    typedef Operand<T, BM, BK, A_KC, PF, KTAIL, NTHR, STREAM == 1 ? kNonTemporal : 0> OpA;
    typedef Operand<T, BN, BK, B_KC, PF, KTAIL, NTHR, STREAM == 2 ? kNonTemporal : 0> OpB;
    typedef Frag<T, NBM, A_KC, OpA::LD, MI> FragA;
    typedef Frag<T, NBN, B_KC, OpB::LD, MI> FragB;

    __shared__ __attribute__((aligned(16))) T smem[2 * (OpA::ELEMS + OpB::ELEMS)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave: scalar
    const int wm0 = (wave / WAVES_N) * WTM;
    const int wn0 = (wave % WAVES_N) * WTN;

    // ---- tile index: XCD-aware remap, then GROUP_M-tall column walk ----
    // Blocks [0, num_full) own whole tiles; the rest are (tile, k-part) units.
    int id = blockIdx.x;
    int part = 0;
    const bool is_split = id >= p.num_full;
    if (is_split) {
        const int u = id - p.num_full;
        id = p.num_full + u / p.split;
        part = u - (u / p.split) * p.split;
    } else if ((p.num_full & 7) == 0) {
        const int per_xcd = p.num_full >> 3;
        id = (id & 7) * per_xcd + (id >> 3);
    }
    int tm, tn;
    tile_coords(p, id, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const T* A;
    const T* B;
    T* C;
    batch_bases(p, (int64_t)blockIdx.z, A, B, C);

    // ---- operand tile bases and extents ----
    // A k-contiguous: element (m, k) at m*lda + k; x-contiguous: at k*lda + m.
    const int64_t a_span = A_KC ? ((int64_t)(p.M - 1) * p.lda + p.K) * (int64_t)sizeof(T)
                                : ((int64_t)(p.K - 1) * p.lda + p.M) * (int64_t)sizeof(T);
    const int64_t b_span = B_KC ? ((int64_t)(p.N - 1) * p.ldb + p.K) * (int64_t)sizeof(T)
                                : ((int64_t)(p.K - 1) * p.ldb + p.N) * (int64_t)sizeof(T);
    const int64_t a_org = A_KC ? (int64_t)m0 * p.lda : (int64_t)m0;  // element offset, tile 0
    const int64_t b_org = B_KC ? (int64_t)n0 * p.ldb : (int64_t)n0;
    const int64_t a_step = A_KC ? BK : (int64_t)BK * p.lda;
    const int64_t b_step = B_KC ? BK : (int64_t)BK * p.ldb;

    OpA opa;
    OpB opb;
    opa.init(tid, p.lda, p.M - m0);
    opb.init(tid, p.ldb, p.N - n0);

    typename MF::acc_t acc[NBM][NBN];
#pragma unroll
    for (int i = 0; i < NBM; ++i)
#pragma unroll
        for (int j = 0; j < NBN; ++j)
#pragma unroll
            for (int r = 0; r < MF::NACC; ++r) acc[i][j][r] = 0;

    // k tiles [kt0, nk) of this block (a k-part for split units)
    const int nk_all = (p.K + BK - 1) / BK;
    const int kt0 = is_split ? (int)((int64_t)part * nk_all / p.split) : 0;
    const int nk = is_split ? (int)((int64_t)(part + 1) * nk_all / p.split) : nk_all;

    // Fixed descriptors at the tile's k = 0 origin, for the k tiles that are
    // full and not the last (see the main loop).  Usable when every offset
    // of the walk over K fits in 31 bits; otherwise every tile takes the
    // moving descriptors of `issue`.
    const __amdgpu_buffer_rsrc_t ra0 = make_rsrc(A + a_org, a_span - a_org * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t rb0 = make_rsrc(B + b_org, b_span - b_org * (int64_t)sizeof(T));
    const int64_t a_tile = A_KC ? (int64_t)BM * p.lda + BK : (int64_t)BK * p.lda + BM;
    const int64_t b_tile = B_KC ? (int64_t)BN * p.ldb + BK : (int64_t)BK * p.ldb + BN;
    const bool fixed_ok = ((int64_t)nk * a_step + a_tile) * (int64_t)sizeof(T) < kMaxRecords - 64 &&
                          ((int64_t)nk * b_step + b_tile) * (int64_t)sizeof(T) < kMaxRecords - 64;
    auto issue_fixed = [&](auto S, int kt) {
        const int k_rem = p.K - kt * BK;
        opa.template load_fixed<decltype(S)::value>(ra0, (int)(kt * a_step * (int64_t)sizeof(T)), k_rem);
        opb.template load_fixed<decltype(S)::value>(rb0, (int)(kt * b_step * (int64_t)sizeof(T)), k_rem);
    };
    // global tile kt -> staging set S
    auto issue = [&](auto S, int kt) {
        const int64_t pa = a_org + kt * a_step, pb = b_org + kt * b_step;
        const int k_rem = p.K - kt * BK;
        opa.template load<decltype(S)::value>(
            make_rsrc(A + pa, a_span - pa * (int64_t)sizeof(T)), k_rem);
        opb.template load<decltype(S)::value>(
            make_rsrc(B + pb, b_span - pb * (int64_t)sizeof(T)), k_rem);
    };
    // staging set S -> LDS buffer buf
    auto commit = [&](auto S, int buf, auto MASK) {
        constexpr bool mask = decltype(MASK)::value;
        opa.template store<decltype(S)::value, mask>(smem + buf * OpA::ELEMS);
        opb.template store<decltype(S)::value, mask>(smem + 2 * OpA::ELEMS + buf * OpB::ELEMS);
    };

    T fa[2][NBM][V], fb[2][NBN][V];  // fragments, double-buffered across k groups
    auto read_frags = [&](auto F, int buf, int g) {
        FragA::read(smem + buf * OpA::ELEMS, wm0, g, lane, fa[decltype(F)::value]);
        FragB::read(smem + 2 * OpA::ELEMS + buf * OpB::ELEMS, wn0, g, lane,
                    fb[decltype(F)::value]);
    };
    auto mma = [&](auto F) {
        constexpr int f = decltype(F)::value;
#pragma unroll
        for (int kk = 0; kk < V; ++kk)
#pragma unroll
            for (int i = 0; i < NBM; ++i)
#pragma unroll
                for (int j = 0; j < NBN; ++j) acc[i][j] = MF::mma(fa[f][i][kk], fb[f][j][kk], acc[i][j]);
    };

    // Instruction counts that the scheduling hints below interleave.
    constexpr int MPG = NBM * NBN * V;  // MFMAs per k group
    // (fragment reads counted as the instructions the compiler emits: a hint
    // pattern that asks for more reads than exist does not take hold)
    constexpr int RPG = FragA::INSTR + FragB::INSTR;
    constexpr int NLD = OpA::NV + OpB::NV;  // global loads (= LDS writes) per tile
    static_assert(G % 2 == 0, "fragment double-buffering needs an even number of k groups");

    // One k tile held in LDS buffer cur, its group-0 fragments already in
    // registers.  Region A: the MFMAs of groups 0..G-2 overlap the fragment
    // reads of groups 1..G-1 and the LDS writes of tile kt + 1.  Then one
    // barrier.  Region B: the MFMAs of the last group overlap the fragment
    // reads of the next tile's group 0.  The global loads of tile kt + PF go
    // at the start of region B when PF > 1 (the LDS writes then wait on loads
    // issued a step earlier; balancing the memory instructions over the two
    // regions was 0.2-1.5 % faster), and at the start of region A when PF ==
    // 1 (their LDS writes come later in the same step).
    // Tile t is staged in register set (t - kt0) % PF, so step S (= (kt -
    // kt0) % PF) loads into set S -- free since tile kt went to LDS -- and
    // stores set (S + 1) % PF, which holds tile kt + 1 (with PF == 1, the
    // tile this step loads).  PF tiles are in flight, so the LDS writes wait
    // on loads issued PF - 1 steps earlier.
    // The loads, LDS writes and next-tile reads are issued unconditionally so
    // that each region is one basic block the scheduling hints can interleave:
    // past the last k tile the buffer loads are masked (k_rem <= 0 or the
    // next part's data) and what they write to the idle LDS buffer is unused.
    auto step = [&](auto S, int kt, int cur, auto MASK, auto FIXED) {
        constexpr int st = decltype(S)::value;
        auto load_next = [&]() {
            if constexpr (decltype(FIXED)::value) issue_fixed(Int<st>{}, kt + PF);
            else issue(Int<st>{}, kt + PF);
        };
        if constexpr (PF == 1) load_next();
#pragma unroll
        for (int g = 0; g + 1 < G; ++g) {
            if (((g + 1) & 1) == 0) read_frags(Int<0>{}, cur, g + 1);
            else read_frags(Int<1>{}, cur, g + 1);
            if ((g & 1) == 0) mma(Int<0>{});
            else mma(Int<1>{});
        }
        commit(Int<(st + 1) % PF>{}, cur ^ 1, MASK);
        // region A: (PF == 1: the loads first,) the fragment reads, then the
        // LDS writes, each memory instruction followed by a slice of the MFMAs
        if constexpr (PF == 1)
            hints_a<0, NLD, (G - 1) * RPG, NLD + (G - 1) * RPG + NLD, (G - 1) * MPG>();
        else
            hints_a<0, 0, (G - 1) * RPG, (G - 1) * RPG + NLD, (G - 1) * MPG>();
        __syncthreads();
        if constexpr (PF > 1) load_next();
        read_frags(Int<0>{}, cur ^ 1, 0);
        mma(Int<1>{});
        // region B: (PF > 1: the loads, then) the next tile's group-0 reads,
        // spread over the last group
        if constexpr (PF == 1)
            hints_b<0, RPG, MPG>();
        else
            hints_a<0, NLD, RPG, NLD + RPG, MPG>();
    };

    // prologue: tile kt0 -> set 0 -> LDS buffer 0; tiles kt0+1 .. kt0+PF-1
    // -> sets 1 .. PF-1
    issue(Int<0>{}, kt0);
    commit(Int<0>{}, 0, std::true_type{});
    if constexpr (PF > 1) issue(Int<1>{}, kt0 + 1);
    if constexpr (PF > 2) issue(Int<2>{}, kt0 + 2);
    if constexpr (PF > 3) issue(Int<3>{}, kt0 + 3);
    __syncthreads();
    read_frags(Int<0>{}, 0, 0);
    probe_mark(p, 0);  // start of the k loop (after the prologue's first tile)

    constexpr std::false_type kNo{};
    constexpr std::true_type kYes{};
    int kt = kt0;
    // Fixed-descriptor section: while every tile a step issues (kt + PF) and
    // stores (kt + 1) is a full k tile other than the last, the loads need
    // no per-step descriptor and no k test (a k-contiguous vector can
    // straddle K, and an x-contiguous one the end of the operand, only in
    // the last k tile).  Measured on 8192^3: 7448 -> 7267 us.
    if (fixed_ok) {
        for (; kt + 2 * PF <= nk - 1; kt += PF) {
            const int cur = (kt - kt0) & 1;
            step(Int<0>{}, kt, cur, kNo, kYes);
            if constexpr (PF > 1) step(Int<1 % PF>{}, kt + 1, cur ^ 1, kNo, kYes);
            if constexpr (PF > 2) step(Int<2 % PF>{}, kt + 2, cur, kNo, kYes);
            if constexpr (PF > 3) step(Int<3 % PF>{}, kt + 3, cur ^ 1, kNo, kYes);
        }
    }
    // the rest with moving descriptors (kt - kt0 is a multiple of PF here)
    if constexpr (!KTAIL) {
        if constexpr (PF == 1) {
            for (; kt < nk; ++kt) step(Int<0>{}, kt, (kt - kt0) & 1, kNo, kNo);
        } else {
            for (; kt < nk; kt += PF) {
                const int cur = (kt - kt0) & 1;
                step(Int<0>{}, kt, cur, kNo, kNo);
                if (kt + 1 < nk) step(Int<1 % PF>{}, kt + 1, cur ^ 1, kNo, kNo);
                if constexpr (PF > 2) {
                    if (kt + 2 < nk) step(Int<2 % PF>{}, kt + 2, cur, kNo, kNo);
                }
                if constexpr (PF > 3) {
                    if (kt + 3 < nk) step(Int<3 % PF>{}, kt + 3, cur ^ 1, kNo, kNo);
                }
            }
        }
    } else {
        // Step kt stores tile kt + 1 to LDS, and only tile nk - 1 can hold
        // a vector that straddles K, so the loop runs its steps unmasked up
        // to step nk - 3 and the remaining steps (fewer than PF + 2) run
        // once, masked, after it: no branch inside the loop.
        for (; kt + PF <= nk - 2; kt += PF) {
            const int cur = (kt - kt0) & 1;
            step(Int<0>{}, kt, cur, kNo, kNo);
            if constexpr (PF > 1) step(Int<1 % PF>{}, kt + 1, cur ^ 1, kNo, kNo);
            if constexpr (PF > 2) step(Int<2 % PF>{}, kt + 2, cur, kNo, kNo);
            if constexpr (PF > 3) step(Int<3 % PF>{}, kt + 3, cur ^ 1, kNo, kNo);
        }
        // the rest, staging sets 0, 1, ... in order
        const int cur = (kt - kt0) & 1;
        if (kt < nk) step(Int<0>{}, kt, cur, kYes, kNo);
        if (kt + 1 < nk) step(Int<1 % PF>{}, kt + 1, cur ^ 1, kYes, kNo);
        if constexpr (PF > 1) {
            if (kt + 2 < nk) step(Int<2 % PF>{}, kt + 2, cur, kYes, kNo);
        }
        if constexpr (PF > 2) {
            if (kt + 3 < nk) step(Int<3 % PF>{}, kt + 3, cur ^ 1, kYes, kNo);
        }
        if constexpr (PF > 3) {
            if (kt + 4 < nk) step(Int<4 % PF>{}, kt + 4, cur, kYes, kNo);
        }
    }

    probe_mark(p, 1);  // end of the k loop

    // ---- epilogue ----
    // Whole tile: C = alpha*acc + beta*C (C is not read when beta == 0).
    // Split unit: the raw fp partial goes to its BM x BN slot of the
    // workspace (row-major, tile-local); splitk_reduce_kernel finishes C.
    // With B n-contiguous, a lane owns UB consecutive columns of each row and
    // writes them with one vector store when the destination allows it.
    constexpr int UB = FragB::U;
    const int q = lane / MB, jl = lane % MB;
    typedef typename Glob<T>::type GT;
    GT* dst;
    int64_t ldd;
    int row_lim, col_lim;
    T alpha, beta;
    bool vec_ok;
    bool relu = false;
    // triangle window of a row: columns [m + lo_off, m + hi_off] of the tile
    // stay (local column c of local row m is global column n0 + c, row m0 + m)
    int lo_off = -(1 << 30), hi_off = 1 << 30;
    if (is_split) {
        // batch entry z's partials follow those of entries 0 .. z-1
        const int64_t slot = (int64_t)blockIdx.z * (p.tiles - p.num_full) + (id - p.num_full);
        dst = (GT*)(p.ws + (slot * p.split + part) * (BM * BN));
        ldd = BN;
        row_lim = BM;
        col_lim = BN;
        alpha = (T)1;
        beta = (T)0;
        vec_ok = true;
    } else {
        dst = (GT*)(C + (int64_t)m0 * p.ldc + n0);
        ldd = p.ldc;
        row_lim = p.M - m0;
        col_lim = p.N - n0;
        alpha = p.alpha;
        beta = p.beta;
        vec_ok = p.c_vec;
        relu = p.relu != 0;
        if (p.uplo == 1) hi_off = m0 - n0;       // column <= row
        else if (p.uplo == 2) lo_off = m0 - n0;  // column >= row
    }
    const bool read_c = beta != (T)0;

    // A wave tile wholly inside C (and inside the triangle window) -- every
    // split unit and every tile of a large problem but the edges -- takes a
    // path without per-element tests: a block row's C loads are all issued
    // before the first of them is used.  Rows that allow vector access use
    // UB-wide loads and stores, others UB single ones.  (Under the general
    // path's per-element branches each load waited for its own round trip
    // before the next was issued: ~18 us per round of 256x256 tiles at
    // 8192^3 with beta != 0.)
    const bool interior = wm0 + WTM <= row_lim && wn0 + WTN <= col_lim &&
                          wn0 + WTN - 1 <= wm0 + hi_off && wn0 >= wm0 + WTM - 1 + lo_off;
    if (interior) {
        constexpr int NS = NBN / UB;
        auto finish = [&](auto WITH_C, auto VEC) {
            typedef typename std::conditional<decltype(VEC)::value, CVec<T, UB>, CElems<T, UB>>::type CV;
#pragma unroll
            for (int i = 0; i < NBM; ++i) {
                T cv[NS][MF::NACC][UB];
                if constexpr (decltype(WITH_C)::value) {
#pragma unroll
                    for (int s = 0; s < NS; ++s)
#pragma unroll
                        for (int r = 0; r < MF::NACC; ++r) {
                            const int m = wm0 + FragA::map(i, MF::row(r, q));
                            const int nb = wn0 + FragB::map(s * UB, jl);
                            CV::load(dst + (int64_t)m * ldd + nb, cv[s][r]);
                        }
                }
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < MF::NACC; ++r) {
                        const int m = wm0 + FragA::map(i, MF::row(r, q));
                        const int nb = wn0 + FragB::map(s * UB, jl);
                        T v[UB];
#pragma unroll
                        for (int u = 0; u < UB; ++u) {
                            v[u] = alpha * acc[i][s * UB + u][r];
                            if constexpr (decltype(WITH_C)::value) v[u] += beta * cv[s][r][u];
                            if (relu) v[u] = relu_of(v[u]);
                        }
                        CV::store(dst + (int64_t)m * ldd + nb, v);
                    }
            }
        };
        if (UB == 1 || vec_ok) {
            if (read_c) finish(Int<1>{}, std::true_type{});
            else finish(Int<0>{}, std::true_type{});
        } else {
            if (read_c) finish(Int<1>{}, std::false_type{});
            else finish(Int<0>{}, std::false_type{});
        }
        return;
    }

#pragma unroll
    for (int i = 0; i < NBM; ++i)
#pragma unroll
        for (int s = 0; s < NBN / UB; ++s) {
            const int nb = wn0 + FragB::map(s * UB, jl);
#pragma unroll
            for (int r = 0; r < MF::NACC; ++r) {
                const int m = wm0 + FragA::map(i, MF::row(r, q));
                if (m >= row_lim) continue;
                const int c_lo = max(0, m + lo_off);
                const int c_hi = min(col_lim, m + hi_off + 1);
                const bool vec = UB > 1 && vec_ok && nb >= c_lo && nb + UB <= c_hi;
                GT* cp = dst + (int64_t)m * ldd + nb;
                T v[UB];
#pragma unroll
                for (int u = 0; u < UB; ++u) v[u] = alpha * acc[i][s * UB + u][r];
                if (vec) {
                    if (read_c) {
                        T c[UB];
                        CVec<T, UB>::load(cp, c);
#pragma unroll
                        for (int u = 0; u < UB; ++u) v[u] += beta * c[u];
                    }
                    if (relu) {
#pragma unroll
                        for (int u = 0; u < UB; ++u) v[u] = relu_of(v[u]);
                    }
                    CVec<T, UB>::store(cp, v);
                } else {
#pragma unroll
                    for (int u = 0; u < UB; ++u)
                        if (nb + u >= c_lo && nb + u < c_hi) {
                            T w = v[u];
                            if (read_c) w += beta * cp[u];
                            cp[u] = relu ? relu_of(w) : w;
                        }
                }
            }
        }
}

// Split-K finish: for tail tile `slot` (tile id num_full + slot), sum the
// `split` partials in part order (deterministic), then C = alpha*sum + beta*C
// (and the ReLU when fused); for a triangle, only the triangle's elements.
// A lane owns RV consecutive elements of a tile row (16 bytes of each
// partial); a workgroup of 256 lanes one 256*RV-element chunk of a tail
// tile.  Partials are read 16 parts at a time, their loads issued before
// the sums; C is read and written with one vector access where its rows
// allow.
constexpr int kMaxSplitParts = 32;

template <typename T, int BM, int BN>
struct SplitReduce {
    static constexpr int RV = 16 / (int)sizeof(T);
    static_assert(BN % RV == 0 && (BM * BN) % (256 * RV) == 0, "tile not divisible over the lanes");
    static constexpr int CHUNKS = BM * BN / (256 * RV);
};

template <typename T, int BM, int BN>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs<T> p)
{
    typedef SplitReduce<T, BM, BN> SR;
    constexpr int RV = SR::RV;
    typedef T vec_t __attribute__((ext_vector_type(RV)));
    typedef typename Glob<vec_t>::type GV;
    typedef typename Glob<T>::type GT;
    const int slot = blockIdx.x / SR::CHUNKS;
    const int chunk = blockIdx.x - slot * SR::CHUNKS;
    int tm, tn;
    tile_coords(p, p.num_full + slot, tm, tn);
    const int e = (chunk * 256 + (int)threadIdx.x) * RV;  // first element, tile-local
    const int m = tm * BM + e / BN;
    const int n = tn * BN + e % BN;
    if (m >= p.M || n >= p.N) return;
    // columns of this lane's run that C (and the triangle window) keeps
    int lo = n, hi = min(p.N, n + RV);  // [lo, hi)
    if (p.uplo == 1) hi = min(hi, m + 1);       // column <= row
    else if (p.uplo == 2) lo = max(lo, m);      // column >= row
    if (lo >= hi) return;
    const int64_t zslot = (int64_t)blockIdx.z * (p.tiles - p.num_full) + slot;
    const GV* part0 = (const GV*)(p.ws + zslot * p.split * (BM * BN) + e);
    constexpr int PV = (BM * BN) / RV;  // vectors per partial
    vec_t sum = part0[0];
    for (int q0 = 1; q0 < p.split; q0 += 16) {
        vec_t v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (q0 + j < p.split) v[j] = part0[(int64_t)(q0 + j) * PV];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (q0 + j < p.split) sum += v[j];
    }
    const T* Az;
    const T* Bz;
    T* Cz;
    batch_bases(p, (int64_t)blockIdx.z, Az, Bz, Cz);
    GT* cp = (GT*)(Cz + (int64_t)m * p.ldc + n);
    const T alpha = p.alpha, beta = p.beta;
    if (p.c_vec && lo == n && hi == n + RV) {
        vec_t out = alpha * sum;
        if (beta != (T)0) out += beta * *(const GV*)cp;
        if (p.relu) {
#pragma unroll
            for (int u = 0; u < RV; ++u) out[u] = relu_of(out[u]);
        }
        *(GV*)cp = out;
        return;
    }
#pragma unroll
    for (int u = 0; u < RV; ++u) {
        if (n + u < lo || n + u >= hi) continue;
        T out = alpha * sum[u];
        if (beta != (T)0) out += beta * cp[u];
        cp[u] = p.relu ? relu_of(out) : out;
    }
}

}  // namespace sbx
