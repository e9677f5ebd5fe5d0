// gemm_aux.hip -- the non-MFMA kernels of the GEMM path:
//   * gemm_generic_kernel: fallback GEMM with 64-bit addressing for shapes
//     the MFMA tiles cannot address with 32-bit buffer offsets (huge leading
//     dimensions); also the independent second path the tests compare the
//     MFMA kernels against.
//   * scale_kernel: the alpha == 0 / k == 0 quick return, C <- beta*C, with
//     beta == 0 writing zeros without reading C (netlib/oneMKL convention for
//     the oneMKL call at src/ops/blas/level3/gemm.cpp:63).
//   * philox fill kernels: synthetic inputs generated directly in HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.hpp"

namespace sbx {

// ---------------------------------------------------------------------------
// Generic GEMM: 64x64 macro tile, 256 lanes, each lane a 4x4 strided patch.
// ---------------------------------------------------------------------------
template <typename T, bool TA, bool TB>
__global__ void __launch_bounds__(256) gemm_generic_kernel(GemmArgs<T> p)
{
    __shared__ T As[16][64 + 1];  // [k][m]
    __shared__ T Bs[16][64 + 1];  // [k][n]
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int tm = blockIdx.x % p.tiles_m, tn = blockIdx.x / p.tiles_m;
    // a triangle (SYRK) skips the tiles wholly outside it
    if ((p.uplo == 1 && tn > tm) || (p.uplo == 2 && tn < tm)) return;
    const int64_t m0 = (int64_t)tm * 64, n0 = (int64_t)tn * 64;
    const T* A;
    const T* B;
    T* C;
    batch_bases(p, (int64_t)blockIdx.z, A, B, C);

    T acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0;

    for (int64_t k0 = 0; k0 < p.K; k0 += 16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = j * 256 + tid;
            // A tile: lanes walk the contiguous index of op(A)'s storage.
            int mm, kk;
            if (TA) { mm = e & 63; kk = e >> 6; } else { kk = e & 15; mm = e >> 4; }
            const int64_t gm = m0 + mm, gk = k0 + kk;
            T va = 0;
            if (gm < p.M && gk < p.K) va = TA ? A[gk * p.lda + gm] : A[gm * p.lda + gk];
            As[kk][mm] = va;
            int nn, kb;
            if (TB) { kb = e & 15; nn = e >> 4; } else { nn = e & 63; kb = e >> 6; }
            const int64_t gn = n0 + nn, gkb = k0 + kb;
            T vb = 0;
            if (gn < p.N && gkb < p.K) vb = TB ? B[gn * p.ldb + gkb] : B[gkb * p.ldb + gn];
            Bs[kb][nn] = vb;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            T a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[k][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
        }
        __syncthreads();
    }

    const bool read_c = p.beta != (T)0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
            const bool in_tri = p.uplo == 0 || (p.uplo == 1 ? n <= m : n >= m);
            if (m < p.M && n < p.N && in_tri) {
                T* cp = C + m * p.ldc + n;
                T v = p.alpha * acc[i][j];
                if (read_c) v += p.beta * *cp;
                *cp = p.relu ? relu_of(v) : v;
            }
        }
}

template <typename T>
hipError_t launch_generic(const GemmArgs<T>& a, bool trans_a, bool trans_b, int batch,
                          hipStream_t stream)
{
    const dim3 grid((unsigned)(a.tiles_m * a.tiles_n), 1, (unsigned)batch);
    const dim3 block(256);
    if (trans_a) {
        if (trans_b) gemm_generic_kernel<T, true, true><<<grid, block, 0, stream>>>(a);
        else gemm_generic_kernel<T, true, false><<<grid, block, 0, stream>>>(a);
    } else {
        if (trans_b) gemm_generic_kernel<T, false, true><<<grid, block, 0, stream>>>(a);
        else gemm_generic_kernel<T, false, false><<<grid, block, 0, stream>>>(a);
    }
    return hipGetLastError();
}

template hipError_t launch_generic<float>(const GemmArgs<float>&, bool, bool, int, hipStream_t);
template hipError_t launch_generic<double>(const GemmArgs<double>&, bool, bool, int,
                                           hipStream_t);

// ---------------------------------------------------------------------------
// C <- beta*C over an m x n row-major window (then the ReLU when fused);
// uplo 1 / 2 restricts it to the lower / upper triangle (SYRK's quick return).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) scale_kernel(T* C, int64_t ldc, int64_t str_c, int64_t m,
                                                    int64_t n, T beta, int relu, int uplo,
                                                    const void* const* table)
{
    T* c = table ? static_cast<T*>(const_cast<void*>(table[3 * (int64_t)blockIdx.z + 2]))
                 : C + (int64_t)blockIdx.z * str_c;
    const int64_t total = m * n;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * 256) {
        const int64_t i = e / n, j = e - i * n;
        if ((uplo == 1 && j > i) || (uplo == 2 && j < i)) continue;
        T* cp = c + i * ldc + j;
        const T v = beta == (T)0 ? (T)0 : beta * *cp;
        *cp = relu ? relu_of(v) : v;
    }
}

template <typename T>
hipError_t launch_scale(T* C, int64_t ldc, int64_t str_c, int64_t m, int64_t n, T beta,
                        int relu, int uplo, int batch, hipStream_t stream,
                        const void* const* table)
{
    int64_t blocks = (m * n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    scale_kernel<T><<<dim3((unsigned)blocks, 1, (unsigned)batch), dim3(256), 0, stream>>>(
        C, ldc, str_c, m, n, beta, relu, uplo, table);
    return hipGetLastError();
}

template hipError_t launch_scale<float>(float*, int64_t, int64_t, int64_t, int64_t, float, int,
                                        int, int, hipStream_t, const void* const*);
template hipError_t launch_scale<double>(double*, int64_t, int64_t, int64_t, int64_t, double,
                                         int, int, int, hipStream_t, const void* const*);

// ---------------------------------------------------------------------------
// Elementwise ReLU over n contiguous elements (the stand-alone form of the
// reference's NonLinearOps::relu, src/ops/math/nonlinear/relu.cpp:38-41).
// HBM bound: 2 * n * sizeof(T) bytes.  16-byte accesses when aligned.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) relu_kernel(T* x, int64_t n)
{
    constexpr int V = 16 / (int)sizeof(T);
    typedef T vec_t __attribute__((ext_vector_type(V)));
    const int64_t nv = ((uintptr_t)x % 16 == 0) ? n / V : 0;
    vec_t* xv = reinterpret_cast<vec_t*>(x);
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv;
         i += (int64_t)gridDim.x * 256) {
        vec_t v = xv[i];
#pragma unroll
        for (int u = 0; u < V; ++u) v[u] = relu_of(v[u]);
        xv[i] = v;
    }
    for (int64_t i = nv * V + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256)
        x[i] = relu_of(x[i]);
}

template <typename T>
hipError_t launch_relu(T* x, int64_t n, hipStream_t stream)
{
    int64_t blocks = (n / (16 / (int64_t)sizeof(T)) + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    relu_kernel<T><<<(unsigned)blocks, 256, 0, stream>>>(x, n);
    return hipGetLastError();
}

template hipError_t launch_relu<float>(float*, int64_t, hipStream_t);
template hipError_t launch_relu<double>(double*, int64_t, hipStream_t);

}  // namespace sbx

// ---------------------------------------------------------------------------
// Philox4x32-10 fills (Salmon et al., SC'11).  Stream layout:
//   key = seed (lo, hi); counter = (block lo, block hi, stream id, 0)
//   f32 uniform [-1,1): element e <- block e/4, word e%4: (w >> 8)*2^-23 - 1
//   f64 uniform [-1,1): element e <- block e/2, words 2(e%2), 2(e%2)+1:
//                       ((w0 >> 5)*2^26 + (w1 >> 6))*2^-52 - 1
//   normal (Box-Muller in double): element e <- block e/2; u1 in (0,1] from
//   words 0,1; u2 in [0,1) from words 2,3; cos for even e, sin for odd e.
// Every uniform value is exact in its type, so host and device agree bit for
// bit; normals agree to within the rounding of log/sqrt/sincos.
// ---------------------------------------------------------------------------
namespace {

__device__ inline void philox_block(uint64_t seed, uint32_t stream, uint64_t block,
                                    uint32_t (&w)[4])
{
    uint32_t c0 = (uint32_t)block, c1 = (uint32_t)(block >> 32), c2 = stream, c3 = 0;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
        const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    w[0] = c0; w[1] = c1; w[2] = c2; w[3] = c3;
}

__device__ inline double u53(uint32_t a, uint32_t b)
{
    return (double)(((uint64_t)(a >> 5) << 26) | (uint64_t)(b >> 6));
}

__global__ void fill_uniform_f32_kernel(float* out, int64_t n, uint64_t seed, uint32_t stream)
{
    for (int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x; b < (n + 3) / 4;
         b += (int64_t)gridDim.x * 256) {
        uint32_t w[4];
        philox_block(seed, stream, (uint64_t)b, w);
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (4 * b + t < n) out[4 * b + t] = (float)(w[t] >> 8) * 0x1p-23f - 1.0f;
    }
}

__global__ void fill_uniform_f64_kernel(double* out, int64_t n, uint64_t seed, uint32_t stream)
{
    for (int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x; b < (n + 1) / 2;
         b += (int64_t)gridDim.x * 256) {
        uint32_t w[4];
        philox_block(seed, stream, (uint64_t)b, w);
#pragma unroll
        for (int t = 0; t < 2; ++t)
            if (2 * b + t < n) out[2 * b + t] = u53(w[2 * t], w[2 * t + 1]) * 0x1p-52 - 1.0;
    }
}

template <typename T>
__global__ void fill_normal_kernel(T* out, int64_t n, uint64_t seed, uint32_t stream,
                                   double scale)
{
    for (int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x; b < (n + 1) / 2;
         b += (int64_t)gridDim.x * 256) {
        uint32_t w[4];
        philox_block(seed, stream, (uint64_t)b, w);
        const double u1 = (u53(w[0], w[1]) + 1.0) * 0x1p-53;
        const double u2 = u53(w[2], w[3]) * 0x1p-53;
        const double r = sqrt(-2.0 * log(u1));
        const double th = 6.283185307179586476925286766559 * u2;
        out[2 * b] = (T)(r * cos(th) * scale);
        if (2 * b + 1 < n) out[2 * b + 1] = (T)(r * sin(th) * scale);
    }
}

unsigned fill_blocks(int64_t items)
{
    int64_t b = (items + 255) / 256;
    if (b > 8192) b = 8192;
    return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

namespace sbx {

hipError_t launch_fill_uniform(int dtype, void* out, int64_t n, uint64_t seed, uint32_t stream,
                               hipStream_t s)
{
    if (dtype == 0)
        fill_uniform_f32_kernel<<<fill_blocks((n + 3) / 4), 256, 0, s>>>((float*)out, n, seed,
                                                                          stream);
    else
        fill_uniform_f64_kernel<<<fill_blocks((n + 1) / 2), 256, 0, s>>>((double*)out, n, seed,
                                                                          stream);
    return hipGetLastError();
}

hipError_t launch_fill_normal(int dtype, void* out, int64_t n, uint64_t seed, uint32_t stream,
                              double scale, hipStream_t s)
{
    if (dtype == 0)
        fill_normal_kernel<float><<<fill_blocks((n + 1) / 2), 256, 0, s>>>((float*)out, n, seed,
                                                                           stream, scale);
    else
        fill_normal_kernel<double><<<fill_blocks((n + 1) / 2), 256, 0, s>>>((double*)out, n,
                                                                            seed, stream, scale);
    return hipGetLastError();
}

}  // namespace sbx
