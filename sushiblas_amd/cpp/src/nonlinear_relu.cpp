// nonlinear_relu.cpp -- NonLinearOps::relu on the gfx950 backend.
//
// Records the same task as the reference (src/ops/math/nonlinear/relu.cpp:38-41
// through nonlinear_internal.hpp:48-90): name and op id "math.nonlinear.relu",
// the storage base pointer as both read and write set.  The closure calls
// sbx_relu (include/sbx.h) on the context's HIP stream.  The task's fusion
// description lets TaskGraph::execute() fold it into a GEMM recorded just
// before it over the same elements.
#include <SushiBLAS/engine.hpp>
#include <SushiBLAS/ops/math/nonlinear.hpp>

#include "../../../include/sbx.h"

namespace SushiBLAS
{
    using namespace SushiRuntime::Graph::Literals;
    using SushiRuntime::Execution::Event;
    using SushiRuntime::Execution::Queue;

    Event NonLinearOps::relu(Tensor& t)
    {
        int dt = -1;
        if (t.dtype == Core::DataType::FLOAT32) dt = SBX_F32;
        else if (t.dtype == Core::DataType::FLOAT64) dt = SBX_F64;
        SB_THROW_IF(dt < 0, "ReLU is provided for FLOAT32 and FLOAT64 tensors only on the "
                            "gfx950 backend.");

        const int64_t size = t.num_elements;
        void* base = t.storage ? t.storage->data_ptr : nullptr;
        std::vector<void*> rw = base ? std::vector<void*>{base} : std::vector<void*>{};

        SushiRuntime::Graph::TaskMetadata meta;
        meta.name = "math.nonlinear.relu";
        meta.task_type = SushiRuntime::Graph::TaskType::MATH_OP;
        meta.op_id = "math.nonlinear.relu"_op;

        SushiRuntime::Graph::FusionHook fusion;
        if (base && size > 0)
        {
            fusion.kind = SushiRuntime::Graph::FusionHook::RELU;
            fusion.base = base;
            fusion.offset_bytes = t.offset_bytes();
            fusion.elements = size;
            fusion.dtype = static_cast<int>(t.dtype);
        }

        void* x = size > 0 ? t.device_data() : nullptr;  // throws without storage
        engine_.get_graph().add_task(meta, rw, rw,
            [=](Queue& q, const std::vector<Event>&) -> Event
            {
                if (size == 0) return Event();
                const int st = sbx_relu(q.native(), dt, x, size);
                SB_THROW_IF(st != SBX_OK, "ReLU over {} elements failed: {}", size,
                            sbx_status_string(st));
                return Event();
            },
            std::move(fusion));
        return Event();
    }
} // namespace SushiBLAS
