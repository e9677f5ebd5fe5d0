// level2_gemv.cpp -- Level2::gemv on the gfx950 backend.
//
// Same validation, parameter derivation and task recording as the reference
// (src/ops/blas/level2/gemv.cpp:65-148): m, n, lda from A's shape and layout,
// vector lengths and increments as utils.hpp:47-60 derives them, the
// "blas.lvl2.gemv" metadata with (transA, alpha, beta).  The recorded closure
// calls sbx_sgemv / sbx_dgemv (include/sbx.h) on the context's HIP stream
// where the reference's gemv_dispatch<T> (gemv.cpp:44-61) calls oneMKL.
#include <SushiBLAS/engine.hpp>
#include <SushiBLAS/ops/blas/level2.hpp>

#include "../../../include/sbx.h"

namespace SushiBLAS
{
    using namespace SushiRuntime::Graph::Literals;
    using SushiRuntime::Execution::Event;
    using SushiRuntime::Execution::Queue;

    namespace
    {
        // Vector length and increment (utils.hpp:47-60): contiguous -> 1,
        // else only a rank-1 view's stride is accepted.
        void vec_params(const Tensor& t, int64_t& n, int64_t& inc)
        {
            n = t.num_elements;
            if (t.is_contiguous())
            {
                inc = 1;
                return;
            }
            SB_THROW_IF(t.rank > 1, "Level 1 BLAS expects contiguous memory for rank > 1 tensors.");
            inc = t.strides[0];
        }
    } // namespace

    Event Level2::gemv(const Tensor& A, const Tensor& x, Tensor& y, bool transA, float alpha,
                       float beta)
    {
        SB_THROW_IF(A.rank < 2, "GEMV requires A to be at least a 2D matrix.");
        SB_THROW_IF(A.dtype != x.dtype || A.dtype != y.dtype, "Data type mismatch in GEMV.");

        const int32_t rA = A.rank;
        const int64_t m = A.shape[rA - 2];
        const int64_t n = A.shape[rA - 1];
        const int64_t lda = (A.layout == Core::Layout::ROW_MAJOR) ? A.shape[rA - 1] : A.shape[rA - 2];

        int64_t nx, incx, ny, incy;
        vec_params(x, nx, incx);
        vec_params(y, ny, incy);
        SB_THROW_IF(nx != (transA ? m : n), "Dimension mismatch for vector x in GEMV.");
        SB_THROW_IF(ny != (transA ? n : m), "Dimension mismatch for vector y in GEMV.");
        SB_THROW_IF(A.dtype == Core::DataType::COMPLEX32 || A.dtype == Core::DataType::COMPLEX64,
                    "GEMV on complex tensors is not provided by the gfx950 backend "
                    "(FLOAT32 and FLOAT64 only).");
        SB_THROW_IF(A.dtype != Core::DataType::FLOAT32 && A.dtype != Core::DataType::FLOAT64,
                    "Unsupported data type for GEMV.");

        std::vector<void*> reads, writes;
        if (A.storage && A.storage->data_ptr) reads.push_back(A.storage->data_ptr);
        if (x.storage && x.storage->data_ptr) reads.push_back(x.storage->data_ptr);
        if (y.storage && y.storage->data_ptr) writes.push_back(y.storage->data_ptr);

        SushiRuntime::Graph::TaskMetadata meta;
        meta.name = "blas.lvl2.gemv";
        meta.task_type = SushiRuntime::Graph::TaskType::MATH_OP;
        meta.op_id = "blas.lvl2.gemv"_op;
        meta.set_param(0, transA);
        meta.set_param(1, alpha);
        meta.set_param(2, beta);

        const int layout = (A.layout == Core::Layout::ROW_MAJOR) ? 0 : 1;
        const int tA = transA ? 1 : 0;
        auto& graph = engine_.get_graph();
        if (A.dtype == Core::DataType::FLOAT32)
        {
            graph.add_task(meta, reads, writes,
                [=, pA = A.device_data_as<float>(), px = x.device_data_as<float>(),
                 py = y.device_data_as<float>()](Queue& q, const std::vector<Event>&) -> Event
                {
                    const int st = sbx_sgemv(q.native(), layout, tA, m, n, alpha, pA, lda, px, incx,
                                             beta, py, incy);
                    SB_THROW_IF(st != SBX_OK, "GEMV [{}x{}] failed: {}", m, n, sbx_status_string(st));
                    return Event();
                });
        }
        else
        {
            graph.add_task(meta, reads, writes,
                [=, alpha_d = static_cast<double>(alpha), beta_d = static_cast<double>(beta),
                 pA = A.device_data_as<double>(), px = x.device_data_as<double>(),
                 py = y.device_data_as<double>()](Queue& q, const std::vector<Event>&) -> Event
                {
                    const int st = sbx_dgemv(q.native(), layout, tA, m, n, alpha_d, pA, lda, px,
                                             incx, beta_d, py, incy);
                    SB_THROW_IF(st != SBX_OK, "GEMV [{}x{}] failed: {}", m, n, sbx_status_string(st));
                    return Event();
                });
        }
        return Event();
    }
} // namespace SushiBLAS
