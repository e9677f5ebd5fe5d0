// gemv.hip -- y = alpha * op(A) * x + beta * y on gfx950 (the arithmetic the
// reference hands to oneMKL's row_major / column_major::gemv,
// src/ops/blas/level2/gemv.cpp:44-61).
//
// GEMV reads every element of A once and does 2 flops per 4 or 8 bytes, so it
// is bound by HBM bandwidth (8 TB/s), not by the matrix cores: the kernels are
// plain vector-load/FMA streams sized to keep enough bytes in flight.  The
// dispatcher maps column-major calls onto row-major ones (a column-major m x n
// A is a row-major n x m A^T), which leaves two shapes of work:
//
//   * rows:  y[i] = sum_j A[i][j] x[j]   (row-major, no transpose).  A group of
//     LPR lanes walks row i with 16-byte loads and reduces with cross-lane
//     shuffles.  LPR (64, 16 or 4) follows the row length so short rows do
//     not idle lanes.
//   * cols:  y[j] = sum_i A[i][j] x[i]   (row-major, transposed).  A workgroup
//     owns a strip of TC*V consecutive columns; TR = 256/TC thread rows walk
//     the matrix rows, then reduce through LDS in a fixed order.
//
// A is read once, with nontemporal loads (it is not reused, so it should not
// displace x and the partials from the caches).
//
// When rows (resp. column strips) alone cannot fill 256 CUs, the reduction
// dimension is cut into `chunks` ranges (grid y); each range writes its
// partial sums to a workspace and gemv_finish_kernel adds them in a fixed
// order and applies alpha and beta.  The result is deterministic: it depends
// on the problem and the chunking, never on scheduling.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv.hpp"

namespace sbx {

namespace {

// 16-byte vectors whose alignment is only the element's: A's rows and x may
// start at any element, so a vector load is well-defined C++ at 4-byte (fp32)
// or 8-byte (fp64) aligned addresses.  gfx950 serves such loads with one
// 16-byte instruction (the device runs in unaligned access mode).
template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
    typedef float type __attribute__((ext_vector_type(4), aligned(4)));
};
template <>
struct Vec16<double> {
    typedef double type __attribute__((ext_vector_type(2), aligned(8)));
};

template <typename T>
__device__ inline T finish(T acc, T alpha, T beta, const T* yp)
{
    T v = alpha * acc;
    if (beta != (T)0) v += beta * *yp;
    return v;
}

// ---- rows: y[i] = alpha * A[i][:] . x + beta * y[i] -----------------------
// grid.x: row groups of 256/LPR rows; grid.y: column chunks of `cw` columns.
// VEC: x is contiguous; A rows and x are read in 16-byte vectors whatever
// their alignment (the device serves unaligned multi-dword loads).
template <typename T, int LPR, bool VEC>
__global__ void __launch_bounds__(256) gemv_rows_kernel(GemvArgs<T> p)
{
    constexpr int V = 16 / (int)sizeof(T);
    typedef typename Vec16<T>::type vec_t;
    const int g = threadIdx.x / LPR, gl = threadIdx.x % LPR;
    const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + g;
    const int64_t c0 = (int64_t)blockIdx.y * p.cw;
    const int64_t c1 = min(c0 + p.cw, p.cols);
    T acc = 0;
    if (row < p.rows) {
        const T* a = p.A + row * p.lda;
        int64_t j = c0;
        if (VEC) {
            const int64_t cv = c0 + (c1 - c0) / V * V;  // vector part of the chunk
            T part[4] = {0, 0, 0, 0};
            int64_t jj = c0 + (int64_t)gl * V;
            // four independent 16-byte loads in flight per lane
            for (; jj + 3 * LPR * V + V <= cv; jj += 4 * LPR * V) {
                vec_t av[4], xv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    av[u] = __builtin_nontemporal_load(
                        reinterpret_cast<const vec_t*>(a + jj + u * LPR * V));
                    xv[u] = *reinterpret_cast<const vec_t*>(p.x + jj + u * LPR * V);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int e = 0; e < V; ++e) part[u] += av[u][e] * xv[u][e];
            }
            for (; jj + V <= cv; jj += LPR * V) {
                const vec_t av = __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(a + jj));
                const vec_t xv = *reinterpret_cast<const vec_t*>(p.x + jj);
#pragma unroll
                for (int e = 0; e < V; ++e) part[0] += av[e] * xv[e];
            }
            acc = (part[0] + part[1]) + (part[2] + part[3]);
            j = cv;
        }
        for (int64_t jj = j + gl; jj < c1; jj += LPR)
            acc += __builtin_nontemporal_load(a + jj) * p.x[jj * p.incx];
    }
    // reduce over the LPR lanes of the group (fixed butterfly order)
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, LPR);
    if (gl != 0 || row >= p.rows) return;
    if (gridDim.y == 1) {
        T* yp = p.y + row * p.incy;
        *yp = finish(acc, p.alpha, p.beta, yp);
    } else {
        p.ws[(int64_t)blockIdx.y * p.rows + row] = acc;
    }
}

// ---- cols: y[j] = alpha * sum_i A[i][j] x[i] + beta * y[j] -----------------
// A workgroup: TC column threads x TR = 256/TC row threads; a column thread
// owns VC consecutive columns (V, read as one 16-byte vector at any row
// alignment; 1 only through the plan's scalar form).  grid.x: column strips
// of TC*VC; grid.y: row chunks of `cw` rows.
template <typename T, int TC, int VC>
__global__ void __launch_bounds__(256) gemv_cols_kernel(GemvArgs<T> p)
{
    constexpr int TR = 256 / TC;
    const int tc = threadIdx.x % TC, tr = threadIdx.x / TC;
    const int64_t col = ((int64_t)blockIdx.x * TC + tc) * VC;
    const int64_t r0 = (int64_t)blockIdx.y * p.cw;
    const int64_t r1 = min(r0 + p.cw, p.rows);
    T acc[VC];
#pragma unroll
    for (int u = 0; u < VC; ++u) acc[u] = 0;
    if (col < p.cols) {
        int64_t i = r0 + tr;
        if (VC > 1) {
            typedef typename Vec16<T>::type vec_t;
            // Whole vectors also for a strip's last, partial group of
            // columns: the elements past the last column are padding or the
            // next row's, and feed only accumulators that are never stored.
            // Only rows whose vector ends inside the matrix take this path
            // (for a partial group: all but the last one or two rows).
            int64_t r_vec = r1;
            if (col + VC > p.cols) {
                const int64_t last = (p.rows - 1) * p.lda + p.cols - 1;  // last element
                const int64_t room = last - (col + VC - 1);
                r_vec = room < 0 ? 0 : min(r1, room / p.lda + 1);
            }
            // four rows in flight per thread
            for (; i + 3 * TR < r_vec; i += 4 * TR) {
                vec_t av[4];
                T xs[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    av[u] = __builtin_nontemporal_load(
                        reinterpret_cast<const vec_t*>(p.A + (i + u * TR) * p.lda + col));
                    xs[u] = p.x[(i + u * TR) * p.incx];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int e = 0; e < VC; ++e) acc[e] += av[u][e] * xs[u];
            }
            for (; i < r_vec; i += TR) {
                const vec_t av =
                    __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(p.A + i * p.lda + col));
                const T xs = p.x[i * p.incx];
#pragma unroll
                for (int e = 0; e < VC; ++e) acc[e] += av[e] * xs;
            }
        }
        {
            // element loads: VC == 1, or the last rows of a partial group
            for (; i < r1; i += TR) {
                const T xs = p.x[i * p.incx];
#pragma unroll
                for (int e = 0; e < VC; ++e)
                    if (col + e < p.cols)
                        acc[e] += __builtin_nontemporal_load(p.A + i * p.lda + col + e) * xs;
            }
        }
    }
    if (TR > 1) {
        // sum the TR row threads of each column in row-thread order
        __shared__ T red[TR][TC * VC + 1];
#pragma unroll
        for (int e = 0; e < VC; ++e) red[tr][tc * VC + e] = acc[e];
        __syncthreads();
        if (tr != 0) return;
#pragma unroll
        for (int e = 0; e < VC; ++e) {
            T s = red[0][tc * VC + e];
            for (int q = 1; q < TR; ++q) s += red[q][tc * VC + e];
            acc[e] = s;
        }
    }
#pragma unroll
    for (int e = 0; e < VC; ++e) {
        const int64_t j = col + e;
        if (j >= p.cols) break;
        if (gridDim.y == 1) {
            T* yp = p.y + j * p.incy;
            *yp = finish(acc[e], p.alpha, p.beta, yp);
        } else {
            p.ws[(int64_t)blockIdx.y * p.cols + j] = acc[e];
        }
    }
}

// ---- finish: y[e] = alpha * sum_c ws[c][e] + beta * y[e] ---------------------
// A workgroup finishes 32 outputs with 8 lane groups: group g adds chunks
// g, g + 8, g + 16, ... in order (loads batched 8 deep so they overlap), then
// the 8 group sums are added in group order.  The order depends only on the
// chunk count, so the result is deterministic; a single lane per output
// adding up to 256 chunks one after another was latency bound (2048^2
// transposed: 37 us, most of it here).
constexpr int kFinishOut = 32, kFinishGroups = 8;

template <typename T>
__global__ void __launch_bounds__(256) gemv_finish_kernel(GemvArgs<T> p, int64_t len, int chunks)
{
    __shared__ T part[kFinishGroups][kFinishOut];
    const int o = threadIdx.x % kFinishOut, g = threadIdx.x / kFinishOut;
    const int64_t e = (int64_t)blockIdx.x * kFinishOut + o;
    T s = 0;  // a group with no chunk leaves 0 here, never read below
    if (e < len && g < chunks) {
        int c = g;
        s = p.ws[(int64_t)c * len + e];
        c += kFinishGroups;
        for (; c + 7 * kFinishGroups < chunks; c += 8 * kFinishGroups) {
            T v[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = p.ws[(int64_t)(c + q * kFinishGroups) * len + e];
#pragma unroll
            for (int q = 0; q < 8; ++q) s += v[q];
        }
        for (; c < chunks; c += kFinishGroups) s += p.ws[(int64_t)c * len + e];
    }
    part[g][o] = s;
    __syncthreads();
    if (g != 0 || e >= len) return;
    T t = part[0][o];
    for (int q = 1; q < kFinishGroups && q < chunks; ++q) t += part[q][o];
    T* yp = p.y + e * p.incy;
    *yp = finish(t, p.alpha, p.beta, yp);
}

template <typename T, int LPR>
hipError_t launch_rows(const GemvArgs<T>& a, bool vec, dim3 grid, hipStream_t s)
{
    if (vec) gemv_rows_kernel<T, LPR, true><<<grid, dim3(256), 0, s>>>(a);
    else gemv_rows_kernel<T, LPR, false><<<grid, dim3(256), 0, s>>>(a);
    return hipGetLastError();
}

template <typename T, int TC>
hipError_t launch_cols(const GemvArgs<T>& a, bool vec, dim3 grid, hipStream_t s)
{
    constexpr int V = 16 / (int)sizeof(T);
    if (vec) gemv_cols_kernel<T, TC, V><<<grid, dim3(256), 0, s>>>(a);
    else gemv_cols_kernel<T, TC, 1><<<grid, dim3(256), 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

template <typename T>
GemvPlan plan_gemv(bool trans, int64_t rows, int64_t cols, bool vec, int cus)
{
    constexpr int V = 16 / (int)sizeof(T);
    // Workgroups wanted before the reduction dimension is cut.  Both forms
    // stream best with few long-lived workgroups (measured, fp32: transposed
    // 16384^2 at 6.3 TB/s with 256 workgroups and 4.8 TB/s with 4096; 256 x
    // 1M untransposed at 6.8 TB/s with 512 and 6.2 TB/s with 2048).
    const int64_t target = trans ? (int64_t)cus : (int64_t)cus * 2;
    GemvPlan pl{};
    pl.trans = trans;
    pl.vec = vec;
    if (!trans) {
        pl.lanes = cols >= 2048 ? 64 : (cols >= 256 ? 16 : 4);
        pl.groups = (rows + (256 / pl.lanes) - 1) / (256 / pl.lanes);
        const int64_t reduce = cols;
        const int64_t unit = (int64_t)pl.lanes * V * 4;  // one unrolled sweep
        int64_t chunks = 1;
        if (pl.groups < target && reduce >= 4 * unit) {
            chunks = (target + pl.groups - 1) / pl.groups;
            const int64_t most = reduce / (2 * unit);
            if (chunks > most) chunks = most;
            if (chunks > 256) chunks = 256;
            if (chunks < 1) chunks = 1;
        }
        int64_t cw = (reduce + chunks - 1) / chunks;
        cw = (cw + unit - 1) / unit * unit;  // chunks start on whole sweeps
        pl.chunks = (int)((reduce + cw - 1) / cw);
        pl.cw = cw;
        pl.out_len = rows;
    } else {
        const int vc = vec ? V : 1;
        const int64_t need = (cols + vc - 1) / vc;  // column threads needed
        int tc = 256;
        while (tc > 1 && tc / 2 >= need) tc /= 2;
        pl.lanes = tc;
        pl.groups = (cols + (int64_t)tc * vc - 1) / ((int64_t)tc * vc);
        const int tr = 256 / tc;
        const int64_t unit = (int64_t)tr * 4;  // rows one unrolled sweep covers
        int64_t chunks = 1;
        if (pl.groups < target && rows >= 4 * unit) {
            chunks = (target + pl.groups - 1) / pl.groups;
            const int64_t most = rows / (2 * unit);
            if (chunks > most) chunks = most;
            if (chunks > 256) chunks = 256;
            if (chunks < 1) chunks = 1;
        }
        int64_t cw = (rows + chunks - 1) / chunks;
        cw = (cw + unit - 1) / unit * unit;
        pl.chunks = (int)((rows + cw - 1) / cw);
        pl.cw = cw;
        pl.out_len = cols;
    }
    if (pl.chunks < 1) pl.chunks = 1;
    if (pl.cw < 1) pl.cw = 1;
    return pl;
}

template <typename T>
hipError_t launch_gemv(GemvArgs<T> a, const GemvPlan& pl, hipStream_t s)
{
    a.cw = pl.cw;
    const dim3 grid((unsigned)pl.groups, (unsigned)pl.chunks, 1);
    hipError_t e;
    if (!pl.trans) {
        switch (pl.lanes) {
        case 64: e = launch_rows<T, 64>(a, pl.vec, grid, s); break;
        case 16: e = launch_rows<T, 16>(a, pl.vec, grid, s); break;
        default: e = launch_rows<T, 4>(a, pl.vec, grid, s); break;
        }
    } else {
        switch (pl.lanes) {
        case 256: e = launch_cols<T, 256>(a, pl.vec, grid, s); break;
        case 128: e = launch_cols<T, 128>(a, pl.vec, grid, s); break;
        case 64: e = launch_cols<T, 64>(a, pl.vec, grid, s); break;
        case 32: e = launch_cols<T, 32>(a, pl.vec, grid, s); break;
        case 16: e = launch_cols<T, 16>(a, pl.vec, grid, s); break;
        case 8: e = launch_cols<T, 8>(a, pl.vec, grid, s); break;
        case 4: e = launch_cols<T, 4>(a, pl.vec, grid, s); break;
        case 2: e = launch_cols<T, 2>(a, pl.vec, grid, s); break;
        default: e = launch_cols<T, 1>(a, pl.vec, grid, s); break;
        }
    }
    if (e != hipSuccess || pl.chunks == 1) return e;
    const int64_t blocks = (pl.out_len + kFinishOut - 1) / kFinishOut;
    gemv_finish_kernel<T><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(a, pl.out_len, pl.chunks);
    return hipGetLastError();
}

template GemvPlan plan_gemv<float>(bool, int64_t, int64_t, bool, int);
template GemvPlan plan_gemv<double>(bool, int64_t, int64_t, bool, int);
template hipError_t launch_gemv<float>(GemvArgs<float>, const GemvPlan&, hipStream_t);
template hipError_t launch_gemv<double>(GemvArgs<double>, const GemvPlan&, hipStream_t);

}  // namespace sbx
