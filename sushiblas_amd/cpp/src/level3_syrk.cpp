// level3_syrk.cpp -- Level3::syrk on the gfx950 backend.
//
// Same validation, parameter derivation and task recording as the reference
// (src/ops/blas/level3/syrk.cpp:84-194): n from the square C, k and the
// inner dimension from A and transA, batch from C's leading dims with
// strides[-3], lda/ldc from the shapes, layout from A, the "blas.lvl3.syrk"
// metadata with (alpha, beta, upper, transA).  The recorded closure calls
// sbx_{s,d}syrk_strided_batched (include/sbx.h) where the reference's
// syrk_dispatch<T> (syrk.cpp:44-79) calls oneMKL.
#include <SushiBLAS/engine.hpp>
#include <SushiBLAS/ops/blas/level3.hpp>

#include "../../../include/sbx.h"

namespace SushiBLAS
{
    using namespace SushiRuntime::Graph::Literals;
    using SushiRuntime::Execution::Event;
    using SushiRuntime::Execution::Queue;

    Event Level3::syrk(const Tensor& A, Tensor& C, bool upper, bool transA, float alpha,
                       float beta)
    {
        SB_THROW_IF(A.rank < 2 || C.rank < 2, "SYRK requires at least 2D tensors.");
        SB_THROW_IF(A.dtype != C.dtype, "Data type mismatch in SYRK operation.");

        const int32_t rA = A.rank, rC = C.rank;
        const int64_t n = C.shape[rC - 2];
        SB_THROW_IF(C.shape[rC - 1] != n, "SYRK requires C to be a square matrix.");
        const int64_t inner_n = transA ? A.shape[rA - 1] : A.shape[rA - 2];
        const int64_t k = transA ? A.shape[rA - 2] : A.shape[rA - 1];
        SB_THROW_IF(inner_n != n, "Dimension mismatch in SYRK: A does not match C dimension.");

        int64_t batch_size = 1;
        for (int i = 0; i < rC - 2; ++i) batch_size *= C.shape[i];

        const int64_t lda = (A.layout == Core::Layout::ROW_MAJOR) ? A.shape[rA - 1] : A.shape[rA - 2];
        const int64_t ldc = (C.layout == Core::Layout::ROW_MAJOR) ? C.shape[rC - 1] : C.shape[rC - 2];
        const int64_t str_a = (batch_size > 1) ? A.strides[rA - 3] : 0;
        const int64_t str_c = (batch_size > 1) ? C.strides[rC - 3] : 0;

        SB_THROW_IF(A.dtype == Core::DataType::HALF || A.dtype == Core::DataType::COMPLEX32 ||
                        A.dtype == Core::DataType::COMPLEX64,
                    "SYRK on this data type is not provided by the gfx950 backend "
                    "(FLOAT32 and FLOAT64 only).");

        std::vector<void*> reads, writes;
        if (A.storage && A.storage->data_ptr) reads.push_back(A.storage->data_ptr);
        if (C.storage && C.storage->data_ptr) writes.push_back(C.storage->data_ptr);

        SushiRuntime::Graph::TaskMetadata meta;
        meta.name = "blas.lvl3.syrk";
        meta.task_type = SushiRuntime::Graph::TaskType::MATH_OP;
        meta.op_id = "blas.lvl3.syrk"_op;
        meta.set_param(0, alpha);
        meta.set_param(1, beta);
        meta.set_param(2, upper);
        meta.set_param(3, transA);

        const int layout = (A.layout == Core::Layout::ROW_MAJOR) ? 0 : 1;
        const int up = upper ? 1 : 0, tA = transA ? 1 : 0;
        auto& graph = engine_.get_graph();
        if (A.dtype == Core::DataType::FLOAT32)
        {
            graph.add_task(meta, reads, writes,
                [=, pA = A.device_data_as<float>(), pC = C.device_data_as<float>()](
                    Queue& q, const std::vector<Event>&) -> Event
                {
                    const int st = sbx_ssyrk_strided_batched(q.native(), layout, up, tA, n, k, alpha,
                                                             pA, lda, str_a, beta, pC, ldc, str_c,
                                                             batch_size);
                    SB_THROW_IF(st != SBX_OK, "SYRK [{}x{}, k {}, batch {}] failed: {}", n, n, k,
                                batch_size, sbx_status_string(st));
                    return Event();
                });
        }
        else if (A.dtype == Core::DataType::FLOAT64)
        {
            graph.add_task(meta, reads, writes,
                [=, alpha_d = static_cast<double>(alpha), beta_d = static_cast<double>(beta),
                 pA = A.device_data_as<double>(), pC = C.device_data_as<double>()](
                    Queue& q, const std::vector<Event>&) -> Event
                {
                    const int st = sbx_dsyrk_strided_batched(q.native(), layout, up, tA, n, k,
                                                             alpha_d, pA, lda, str_a, beta_d, pC,
                                                             ldc, str_c, batch_size);
                    SB_THROW_IF(st != SBX_OK, "SYRK [{}x{}, k {}, batch {}] failed: {}", n, n, k,
                                batch_size, sbx_status_string(st));
                    return Event();
                });
        }
        else
        {
            SB_THROW_IF(true, "Unsupported data type for SYRK operation.");
        }
        return Event();
    }
} // namespace SushiBLAS
