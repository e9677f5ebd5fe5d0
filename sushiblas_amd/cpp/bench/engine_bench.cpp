// engine_bench.cpp -- times the C++ Engine path (Level3::gemm / NonLinearOps::relu
// recorded into the TaskGraph, then Engine::execute()) on the reference's
// integration patterns, tests/runtime/test_framework_sim.cpp:
//   parallel_inference: 24 independent (256x256)x(256x512) GEMM + ReLU (:75-128)
//   deep_forward:       10 chained (512x1024)x(1024x1024) GEMM + ReLU (:10-73)
//   shard_collision:    3000 independent 8x8 GEMMs (test_dependency_stress.cpp:59-95)
// Tensors are DEVICE allocations filled once, so a step is recording plus
// execution of one batch; each pattern runs with 1 lane (strictly in order)
// and with every lane of the context.  One JSON line per pattern and lane
// count: {"pattern", "lanes", "us_per_batch", "tasks"}.
#include <SushiBLAS/SushiBLAS.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace
{
    using Clock = std::chrono::steady_clock;
    using sb::Core::DataType;
    using SushiRuntime::Memory::AllocStrategy;

    sb::Tensor device_tensor(sb::Engine& e, std::initializer_list<int64_t> dims, float value)
    {
        auto t = e.create_tensor(dims, DataType::FLOAT32, AllocStrategy::DEVICE);
        std::vector<float> v(static_cast<size_t>(t.num_elements), value);
        t.storage->copy_from_host(v.data(), v.size() * sizeof(float));
        return t;
    }

    template <typename Record>
    void time_pattern(const char* name, sb::Engine& e, int tasks, Record record, int reps)
    {
        for (size_t lanes : {size_t(1), SushiRuntime::Execution::RuntimeContext::kLanes})
        {
            e.get_graph().set_max_lanes(lanes);
            for (int w = 0; w < 3; ++w)
            {
                record();
                e.execute().wait();
            }
            const auto t0 = Clock::now();
            for (int r = 0; r < reps; ++r)
            {
                record();
                e.execute().wait();
            }
            const double us =
                std::chrono::duration<double, std::micro>(Clock::now() - t0).count() / reps;
            std::printf("{\"pattern\": \"%s\", \"lanes\": %zu, \"us_per_batch\": %.1f, \"tasks\": %d}\n",
                        name, lanes, us, tasks);
            std::fflush(stdout);
        }
    }
} // namespace

int main()
{
    SushiRuntime::Execution::RuntimeContext ctx;
    sb::Engine engine(ctx);

    {
        const int models = 24, m = 256, n = 512, k = 256;
        std::vector<sb::Tensor> X, W, Y;
        for (int i = 0; i < models; ++i)
        {
            X.push_back(device_tensor(engine, {m, k}, 1.0f));
            W.push_back(device_tensor(engine, {k, n}, 2.0f));
            Y.push_back(device_tensor(engine, {m, n}, 0.0f));
        }
        time_pattern("parallel_inference", engine, 2 * models, [&] {
            for (int i = 0; i < models; ++i)
            {
                engine.blas().gemm(X[i], W[i], Y[i]);
                engine.nonlinear().relu(Y[i]);
            }
        }, 50);
    }
    {
        const int layers = 10, b = 512, f = 1024;
        std::vector<sb::Tensor> H{device_tensor(engine, {b, f}, 1.0f)}, W;
        for (int i = 0; i < layers; ++i)
        {
            W.push_back(device_tensor(engine, {f, f}, 0.01f));
            H.push_back(device_tensor(engine, {b, f}, 0.0f));
        }
        time_pattern("deep_forward", engine, 2 * layers - 1, [&] {
            for (int i = 0; i < layers; ++i)
            {
                engine.blas().gemm(H[i], W[i], H[i + 1]);
                if (i < layers - 1) engine.nonlinear().relu(H[i + 1]);
            }
        }, 50);
    }
    {
        const int ops = 3000, n = 8;
        std::vector<sb::Tensor> A, B, C;
        for (int i = 0; i < ops; ++i)
        {
            A.push_back(device_tensor(engine, {n, n}, float(i % 7)));
            B.push_back(device_tensor(engine, {n, n}, 1.0f));
            C.push_back(device_tensor(engine, {n, n}, 0.0f));
        }
        time_pattern("shard_collision", engine, ops, [&] {
            for (int i = 0; i < ops; ++i) engine.blas().gemm(A[i], B[i], C[i]);
        }, 5);
    }
    return 0;
}
