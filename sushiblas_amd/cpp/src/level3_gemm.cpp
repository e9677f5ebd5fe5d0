// level3_gemm.cpp -- Level3::gemm on the gfx950 backend.
//
// Same validation, parameter derivation and task recording as the reference
// (src/ops/blas/level3/gemm.cpp:82-198): m, n, k, batch, leading dimensions
// from the SHAPES, batch strides strides[r-3], layout taken from A, read and
// write sets from the storage base pointers, the "blas.lvl3.gemm" metadata.
// The recorded closure calls the C ABI (include/sbx.h) on the context's HIP
// stream where the reference's gemm_dispatch<T> (gemm.cpp:44-79) calls oneMKL.
// The task also carries a fusion description (its output run and a ReLU-fused
// form of the same work), which TaskGraph::execute() uses when a ReLU over
// exactly that run is recorded next, and a grouping description (launch
// parameters, operand addresses and a grouped launcher) that lets execute()
// issue a run of independent same-shaped GEMMs as one launch.
#include <SushiBLAS/engine.hpp>
#include <SushiBLAS/ops/blas/level3.hpp>

#include "../../../include/sbx.h"

#include <cstring>

namespace SushiBLAS
{
    using namespace SushiRuntime::Graph::Literals;
    using SushiRuntime::Execution::Event;
    using SushiRuntime::Execution::Queue;

    namespace
    {
        const char* dtype_name(Core::DataType t)
        {
            switch (t)
            {
                case Core::DataType::HALF: return "HALF";
                case Core::DataType::FLOAT32: return "FLOAT32";
                case Core::DataType::FLOAT64: return "FLOAT64";
                case Core::DataType::COMPLEX32: return "COMPLEX32";
                case Core::DataType::COMPLEX64: return "COMPLEX64";
            }
            return "?";
        }
    } // namespace

    Event Level3::gemm(const Tensor& A, const Tensor& B, Tensor& C, bool transA, bool transB,
                       float alpha, float beta)
    {
        SB_THROW_IF(A.rank < 2 || B.rank < 2 || C.rank < 2, "GEMM requires at least 2D tensors.");
        SB_THROW_IF(A.dtype != B.dtype || A.dtype != C.dtype, "Data type mismatch in GEMM operation.");

        const int32_t rA = A.rank, rB = B.rank, rC = C.rank;
        const int64_t m = C.shape[rC - 2];
        const int64_t n = C.shape[rC - 1];
        const int64_t k = transA ? A.shape[rA - 2] : A.shape[rA - 1];

        int64_t batch_size = 1;
        for (int i = 0; i < rC - 2; ++i) batch_size *= C.shape[i];

        const int64_t lda = (A.layout == Core::Layout::ROW_MAJOR) ? A.shape[rA - 1] : A.shape[rA - 2];
        const int64_t ldb = (B.layout == Core::Layout::ROW_MAJOR) ? B.shape[rB - 1] : B.shape[rB - 2];
        const int64_t ldc = (C.layout == Core::Layout::ROW_MAJOR) ? C.shape[rC - 1] : C.shape[rC - 2];

        const int64_t str_a = (batch_size > 1) ? A.strides[rA - 3] : 0;
        const int64_t str_b = (batch_size > 1) ? B.strides[rB - 3] : 0;
        const int64_t str_c = (batch_size > 1) ? C.strides[rC - 3] : 0;

        const int layout = (A.layout == Core::Layout::ROW_MAJOR) ? 0 : 1;
        const int tA = transA ? 1 : 0, tB = transB ? 1 : 0;

        std::vector<void*> reads, writes;
        if (A.storage && A.storage->data_ptr) reads.push_back(A.storage->data_ptr);
        if (B.storage && B.storage->data_ptr) reads.push_back(B.storage->data_ptr);
        if (C.storage && C.storage->data_ptr) writes.push_back(C.storage->data_ptr);

        SushiRuntime::Graph::TaskMetadata meta;
        meta.name = "blas.lvl3.gemm";
        meta.task_type = SushiRuntime::Graph::TaskType::MATH_OP;
        meta.op_id = "blas.lvl3.gemm"_op;
        meta.set_param(0, alpha);
        meta.set_param(1, beta);
        meta.set_param(2, transA);
        meta.set_param(3, transB);

        // The elements this GEMM writes: batch blocks of m*n (ldc is the
        // shape's own extent), one contiguous run when the blocks abut.  A ReLU
        // recorded right after it over exactly that run may be fused into it.
        SushiRuntime::Graph::FusionHook fusion;
        const bool one_run = batch_size == 1 || str_c == m * n;
        if (one_run && C.storage && C.storage->data_ptr && m > 0 && n > 0)
        {
            fusion.kind = SushiRuntime::Graph::FusionHook::PRODUCER;
            fusion.base = C.storage->data_ptr;
            fusion.offset_bytes = C.offset_bytes();
            fusion.elements = batch_size * m * n;
            fusion.dtype = static_cast<int>(C.dtype);
            fusion.fused_name = "blas.lvl3.gemm+relu";
        }

        // Unbatched FLOAT32/FLOAT64 GEMMs may be issued together with other
        // tasks of equal launch parameters (one grouped launch over a table of
        // operand pointers); the key holds every parameter but the pointers.
        SushiRuntime::Graph::GroupHook group;
        if (batch_size == 1 && (A.dtype == Core::DataType::FLOAT32 || A.dtype == Core::DataType::FLOAT64) &&
            A.storage && B.storage && C.storage && m > 0 && n > 0)
        {
            const int dt = A.dtype == Core::DataType::FLOAT32 ? SBX_F32 : SBX_F64;
            uint32_t ab, bb;
            std::memcpy(&ab, &alpha, 4);
            std::memcpy(&bb, &beta, 4);
            group.enabled = true;
            group.key[0] = uint64_t(dt) | uint64_t(layout) << 8 | uint64_t(tA) << 9 | uint64_t(tB) << 10;
            group.key[1] = uint64_t(m);
            group.key[2] = uint64_t(n);
            group.key[3] = uint64_t(k);
            group.key[4] = uint64_t(lda);
            group.key[5] = uint64_t(ldb);
            group.key[6] = uint64_t(ldc);
            group.key[7] = uint64_t(ab) << 32 | bb;
            group.ptrs[0] = A.device_data();
            group.ptrs[1] = B.device_data();
            group.ptrs[2] = C.device_data();
            group.aligned = true;
            for (const void* ptr : group.ptrs) group.aligned = group.aligned && (uintptr_t)ptr % 16 == 0;
            group.launch = [=](Queue& q, const void* const* table, int64_t count, bool aligned,
                               int epilogue) {
                const double ad = alpha, bd = beta;
                const void* pa = dt == SBX_F32 ? static_cast<const void*>(&alpha) : &ad;
                const void* pb = dt == SBX_F32 ? static_cast<const void*>(&beta) : &bd;
                const int st = sbx_gemm_grouped(q.native(), dt, layout, tA, tB, m, n, k, pa, lda, ldb,
                                                pb, ldc, table, count, aligned ? 1 : 0, epilogue);
                SB_THROW_IF(st != SBX_OK, "grouped GEMM [{}x{}x{}, {} problems] failed: {}", m, n, k,
                            count, sbx_status_string(st));
            };
        }

        auto& graph = engine_.get_graph();
        switch (A.dtype)
        {
            case Core::DataType::FLOAT32:
            {
                auto work = [=, pA = A.device_data_as<float>(), pB = B.device_data_as<float>(),
                             pC = C.device_data_as<float>()](int epilogue)
                {
                    return [=](Queue& q, const std::vector<Event>&) -> Event
                    {
                        const int st = sbx_gemm_fused(q.native(), SBX_F32, layout, tA, tB, m, n, k,
                                                      &alpha, pA, lda, str_a, pB, ldb, str_b, &beta,
                                                      pC, ldc, str_c, batch_size, epilogue);
                        SB_THROW_IF(st != SBX_OK, "GEMM [{}x{}x{}, batch {}] failed: {}", m, n, k,
                                    batch_size, sbx_status_string(st));
                        return Event();
                    };
                };
                if (fusion.kind != SushiRuntime::Graph::FusionHook::NONE)
                    fusion.with_relu = work(SBX_EPILOGUE_RELU);
                graph.add_task(meta, reads, writes, work(SBX_EPILOGUE_NONE), std::move(fusion),
                               group);
                break;
            }
            case Core::DataType::FLOAT64:
            {
                auto work = [=, alpha_d = static_cast<double>(alpha),
                             beta_d = static_cast<double>(beta), pA = A.device_data_as<double>(),
                             pB = B.device_data_as<double>(),
                             pC = C.device_data_as<double>()](int epilogue)
                {
                    return [=](Queue& q, const std::vector<Event>&) -> Event
                    {
                        const int st = sbx_gemm_fused(q.native(), SBX_F64, layout, tA, tB, m, n, k,
                                                      &alpha_d, pA, lda, str_a, pB, ldb, str_b,
                                                      &beta_d, pC, ldc, str_c, batch_size, epilogue);
                        SB_THROW_IF(st != SBX_OK, "GEMM [{}x{}x{}, batch {}] failed: {}", m, n, k,
                                    batch_size, sbx_status_string(st));
                        return Event();
                    };
                };
                if (fusion.kind != SushiRuntime::Graph::FusionHook::NONE)
                    fusion.with_relu = work(SBX_EPILOGUE_RELU);
                graph.add_task(meta, reads, writes, work(SBX_EPILOGUE_NONE), std::move(fusion),
                               group);
                break;
            }
            case Core::DataType::HALF:
            case Core::DataType::COMPLEX32:
            case Core::DataType::COMPLEX64:
                SB_THROW_IF(true, "GEMM on {} is not provided by the gfx950 backend "
                                  "(FLOAT32 and FLOAT64 only).", dtype_name(A.dtype));
                break;
            default:
                SB_THROW_IF(true, "Unsupported data type for GEMM operation.");
        }
        return Event();
    }
} // namespace SushiBLAS
