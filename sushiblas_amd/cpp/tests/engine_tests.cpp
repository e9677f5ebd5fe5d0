// engine_tests.cpp -- tests of the C++ Engine/Tensor/Storage/Level3::gemm layer.
//
// The GEMM cases mirror the reference's own tests: tests/blas/level3/test_gemm.cpp
// (known answers), tests/runtime/test_framework_sim.cpp (checked here by value
// through closed forms, where the reference checks only shapes) and
// tests/runtime/test_dependency_stress.cpp (same fan-out; values checked too).
// GoogleTest is not available, so a minimal runner stands in: each case is
// "cpu" (no device needed) or "gpu"; `--cpu`, `--gpu` or case names select.
// Output: one "[  OK  ] name", "[ SKIP ] name: reason" or "[FAILED] name:
// reason" line per case; the exit status is the number of failed cases.
// Cases that read fixtures written by numpy take their directory from
// $SBX_NPY_DIR (tests/test_npy_io.py sets it) and report SKIP without it.
#include <SushiBLAS/SushiBLAS.h>

#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <limits>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

namespace
{
    struct Failure
    {
        std::string what;
    };

    // A case whose inputs are not available (e.g. a fixture directory that
    // the Python driver provides) reports SKIP instead of running.
    struct Skip
    {
        std::string why;
    };

    struct Case
    {
        const char* name;
        bool gpu;
        std::function<void()> fn;
    };

    std::vector<Case>& registry()
    {
        static std::vector<Case> r;
        return r;
    }

    struct Register
    {
        Register(const char* name, bool gpu, std::function<void()> fn)
        {
            registry().push_back({name, gpu, std::move(fn)});
        }
    };

#define TEST_CASE(name, gpu)                                  \
    static void name();                                       \
    static Register reg_##name(#name, gpu, name);             \
    static void name()

#define CHECK(cond)                                                                        \
    do                                                                                     \
    {                                                                                      \
        if (!(cond))                                                                       \
        {                                                                                  \
            std::ostringstream os_;                                                        \
            os_ << __FILE__ << ":" << __LINE__ << ": CHECK(" #cond ") failed";             \
            throw Failure{os_.str()};                                                      \
        }                                                                                  \
    } while (0)

#define CHECK_NEAR(a, b, tol)                                                              \
    do                                                                                     \
    {                                                                                      \
        const double a_ = (a), b_ = (b);                                                   \
        if (!(std::fabs(a_ - b_) <= (tol)))                                                \
        {                                                                                  \
            std::ostringstream os_;                                                        \
            os_ << __FILE__ << ":" << __LINE__ << ": " #a " = " << a_ << " vs " #b " = " << b_; \
            throw Failure{os_.str()};                                                      \
        }                                                                                  \
    } while (0)

#define CHECK_THROWS(stmt)                                                                 \
    do                                                                                     \
    {                                                                                      \
        bool thrown_ = false;                                                              \
        try { stmt; } catch (const std::runtime_error&) { thrown_ = true; }                \
        if (!thrown_) throw Failure{std::string(__FILE__) + ": expected a throw: " #stmt}; \
    } while (0)

    using sb::Core::DataType;
    using sb::Core::Layout;
    using sr::Memory::AllocStrategy;

    // One device context per process, as the reference's fixture holds one
    // static RuntimeContext (tests/test_common.hpp:15).
    sr::Execution::RuntimeContext& ctx()
    {
        static sr::Execution::RuntimeContext c;
        return c;
    }

    template <typename T = float>
    void fill_tensor(sb::Tensor& t, const std::vector<T>& data)
    {
        CHECK(static_cast<int64_t>(data.size()) == t.num_elements);
        std::memcpy(t.data_as<T>(), data.data(), data.size() * sizeof(T));
    }

    template <typename T = float>
    void verify_tensor(const sb::Tensor& t, const std::vector<T>& expected, double abs_error = 1e-4)
    {
        CHECK(static_cast<int64_t>(expected.size()) == t.num_elements);
        const T* p = t.data_as<T>();
        for (size_t i = 0; i < expected.size(); ++i) CHECK_NEAR(p[i], expected[i], abs_error);
    }
} // namespace

// ---------------------------------------------------------------- host only

TEST_CASE(TensorStridesRowAndColumnMajor, false)
{
    sb::Tensor r(nullptr, {2, 3, 4});
    CHECK(r.rank == 3 && r.num_elements == 24);
    CHECK(r.strides[0] == 12 && r.strides[1] == 4 && r.strides[2] == 1);
    sb::Tensor c(nullptr, {2, 3, 4}, 0, Layout::COLUMN_MAJOR);
    CHECK(c.strides[0] == 1 && c.strides[1] == 2 && c.strides[2] == 6);
    CHECK(r.is_contiguous() && c.is_contiguous());
    CHECK(!r.transpose(0, 2).is_contiguous());
    CHECK_THROWS(sb::Tensor(nullptr, {1, 1, 1, 1, 1, 1, 1}));
}

TEST_CASE(TensorViews, false)
{
    sb::Tensor t(nullptr, {4, 6});
    sb::Tensor tt = t.transpose(0, 1);
    CHECK(tt.shape[0] == 6 && tt.shape[1] == 4 && tt.strides[0] == 1 && tt.strides[1] == 6);
    CHECK_THROWS(t.transpose(0, 2));
    sb::Tensor s = t.slice(0, 1, -1);  // rows [1, 3)
    CHECK(s.shape[0] == 2 && s.shape[1] == 6 && s.storage_offset == 6);
    sb::Tensor s2 = t.slice(1, -100, 100);  // clamped
    CHECK(s2.shape[1] == 6 && s2.storage_offset == 0);
    t.dtype = DataType::FLOAT64;
    sb::Tensor r = t.reshape({3, 8});
    CHECK(r.shape[0] == 3 && r.shape[1] == 8 && r.dtype == DataType::FLOAT64);
    CHECK_THROWS(t.reshape({5, 5}));
    CHECK_THROWS(tt.reshape({24}));
}

TEST_CASE(OpIdIsFnv1a, false)
{
    using namespace sr::Graph::Literals;
    CHECK(("blas.lvl3.gemm"_op).value == 0xaea52978u);
    CHECK(sr::Graph::OpID::hash_str("", 0) == 2166136261u);
    sr::Graph::TaskMetadata m;
    m.set_param(0, 1.5f);
    m.set_param(2, true);
    CHECK(m.get_param<float>(0) == 1.5f && m.get_param<bool>(2));
}

TEST_CASE(ErrorFormatting, false)
{
    CHECK(sb::Core::format("a {} b {} c", 1, "x") == "a 1 b x c");
    CHECK(sb::Core::format("no args") == "no args");
    bool thrown = false;
    try { SB_THROW_IF(true, "value {}", 42); }
    catch (const std::runtime_error& e) { thrown = std::string(e.what()) == "value 42"; }
    CHECK(thrown);
}

TEST_CASE(GemmValidationThrowsAtRecordTime, false)
{
    // An Engine over a context that has not touched the device yet: gemm()
    // validates before it needs any allocation (gemm.cpp:87-88).
    sr::Execution::RuntimeContext local;
    sb::Engine e(local);
    sb::Tensor a1(nullptr, {4});
    sb::Tensor a2(nullptr, {4, 4});
    sb::Tensor b2(nullptr, {4, 4});
    sb::Tensor c2(nullptr, {4, 4});
    CHECK_THROWS(e.blas().gemm(a1, b2, c2));
    sb::Tensor d2(nullptr, {4, 4});
    d2.dtype = DataType::FLOAT64;
    CHECK_THROWS(e.blas().gemm(a2, d2, c2));
    sb::Tensor h(nullptr, {4, 4});
    h.dtype = DataType::HALF;
    sb::Tensor h2 = h, h3 = h;
    CHECK_THROWS(e.blas().gemm(h, h2, h3));       // not provided by this backend
    CHECK_THROWS(e.blas().gemm(a2, b2, c2));      // no storage: data() throws at capture
    CHECK(e.get_graph().pending() == 0);
}

TEST_CASE(SushiPtrRefCounting, false)
{
    struct Obj : sr::Core::RefCounted
    {
        int* alive;
        explicit Obj(int* a) : alive(a) { ++*alive; }
        ~Obj() override { --*alive; }
    };
    int alive = 0;
    {
        sr::sushi_ptr<Obj> a = sr::make_sushi<Obj>(&alive);
        CHECK(alive == 1 && a->ref_count() == 1);
        sr::sushi_ptr<Obj> b = a;
        CHECK(a->ref_count() == 2);
        b.reset();
        CHECK(a->ref_count() == 1);
    }
    CHECK(alive == 0);
}

// ------------------------------------------------------------------ device

TEST_CASE(SimpleGEMM3x3, true)  // tests/blas/level3/test_gemm.cpp:39-63
{
    sb::Engine engine(ctx(), Layout::ROW_MAJOR);
    const int N = 3;
    auto A = engine.create_tensor({N, N});
    auto B = engine.create_tensor({N, N});
    auto C = engine.create_tensor({N, N});
    fill_tensor(A, {1, 2, 3, 4, 5, 6, 7, 8, 9});
    fill_tensor(B, {2, 0, 0, 0, 2, 0, 0, 0, 2});
    fill_tensor(C, std::vector<float>(N * N, 0.0f));
    engine.blas().gemm(A, B, C);
    engine.execute().wait();
    verify_tensor(C, {2, 4, 6, 8, 10, 12, 14, 16, 18});
}

TEST_CASE(SimpleGEMMColumnMajor, true)  // tests/blas/level3/test_gemm.cpp:65-88
{
    sb::Engine engine(ctx(), Layout::COLUMN_MAJOR);
    auto A = engine.create_tensor({2, 2});
    auto B = engine.create_tensor({2, 2});
    auto C = engine.create_tensor({2, 2});
    fill_tensor(A, {1, 3, 2, 4});
    fill_tensor(B, {5, 7, 6, 8});
    engine.blas().gemm(A, B, C);
    engine.execute().wait();
    verify_tensor(C, {19, 43, 22, 50});
}

TEST_CASE(DeferredUntilExecute, true)
{
    sb::Engine engine(ctx());
    auto A = engine.create_tensor({2, 2});
    auto B = engine.create_tensor({2, 2});
    auto C = engine.create_tensor({2, 2});
    fill_tensor(A, {1, 2, 3, 4});
    fill_tensor(B, {1, 0, 0, 1});
    fill_tensor(C, {-1, -1, -1, -1});
    sr::Execution::Event ev = engine.blas().gemm(A, B, C);
    CHECK(ev.is_complete());                 // default event, as the reference returns
    CHECK(engine.get_graph().pending() == 1);
    ctx().wait_all();
    verify_tensor(C, {-1, -1, -1, -1});       // nothing ran yet
    engine.execute().wait();
    verify_tensor(C, {1, 2, 3, 4});
    CHECK(engine.get_graph().pending() == 0);
}

TEST_CASE(AlphaBetaTransposesFp32AndFp64, true)
{
    // op(A) = A^T with A stored 3x2 (k x m), op(B) = B^T with B stored 2x3 (n x k)
    sb::Engine engine(ctx());
    for (DataType dt : {DataType::FLOAT32, DataType::FLOAT64})
    {
        auto A = engine.create_tensor({3, 2}, dt);
        auto B = engine.create_tensor({2, 3}, dt);
        auto C = engine.create_tensor({2, 2}, dt);
        const std::vector<double> a = {1, 2, 3, 4, 5, 6}, b = {1, 0, 2, 0, 1, 3}, c = {1, 1, 1, 1};
        // op(A) = [[1,3,5],[2,4,6]], op(B) = [[1,0],[0,1],[2,3]] -> op(A)op(B) = [[11,18],[14,22]]
        const std::vector<double> want = {2 * 11 - 1, 2 * 18 - 1, 2 * 14 - 1, 2 * 22 - 1};
        if (dt == DataType::FLOAT32)
        {
            fill_tensor(A, std::vector<float>(a.begin(), a.end()));
            fill_tensor(B, std::vector<float>(b.begin(), b.end()));
            fill_tensor(C, std::vector<float>(c.begin(), c.end()));
        }
        else
        {
            fill_tensor(A, a);
            fill_tensor(B, b);
            fill_tensor(C, c);
        }
        engine.blas().gemm(A, B, C, true, true, 2.0f, -1.0f);
        engine.execute().wait();
        if (dt == DataType::FLOAT32) verify_tensor(C, std::vector<float>(want.begin(), want.end()));
        else verify_tensor(C, want, 1e-12);
    }
}

TEST_CASE(BatchedRank3, true)  // rank > 2 -> gemm_batch (gemm.cpp:55-58)
{
    sb::Engine engine(ctx());
    const int batch = 4, m = 5, n = 3, k = 7;
    auto A = engine.create_tensor({batch, m, k});
    auto B = engine.create_tensor({batch, k, n});
    auto C = engine.create_tensor({batch, m, n});
    std::vector<float> a(batch * m * k), b(batch * k * n);
    for (size_t i = 0; i < a.size(); ++i) a[i] = float((i * 7) % 11) - 5.0f;
    for (size_t i = 0; i < b.size(); ++i) b[i] = float((i * 5) % 13) - 6.0f;
    fill_tensor(A, a);
    fill_tensor(B, b);
    engine.blas().gemm(A, B, C);
    engine.execute().wait();
    std::vector<float> want(batch * m * n, 0.0f);
    for (int z = 0; z < batch; ++z)
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j)
            {
                double s = 0;
                for (int p = 0; p < k; ++p) s += a[z * m * k + i * k + p] * b[z * k * n + p * n + j];
                want[z * m * n + i * n + j] = float(s);
            }
    verify_tensor(C, want);  // small integers: exact
}

TEST_CASE(SlicedOutputRows, true)
{
    // C is rows [2, 5) of a 6x4 tensor: the view's offset is applied to the
    // device address, rows outside the slice stay untouched.
    sb::Engine engine(ctx());
    auto A = engine.create_tensor({3, 2});
    auto B = engine.create_tensor({2, 4});
    auto Cfull = engine.create_tensor({6, 4});
    fill_tensor(A, {1, 2, 3, 4, 5, 6});
    fill_tensor(B, {1, 0, 1, 0, 0, 1, 0, 1});
    fill_tensor(Cfull, std::vector<float>(24, 9.0f));
    sb::Tensor C = Cfull.slice(0, 2, 5);
    engine.blas().gemm(A, B, C);
    engine.execute().wait();
    std::vector<float> want(24, 9.0f);
    const float rows[3][4] = {{1, 2, 1, 2}, {3, 4, 3, 4}, {5, 6, 5, 6}};
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 4; ++j) want[(i + 2) * 4 + j] = rows[i][j];
    verify_tensor(Cfull, want);
}

TEST_CASE(DeviceStrategyWithExplicitStaging, true)
{
    sb::Engine engine(ctx());
    const int n = 64;
    auto A = engine.create_tensor({n, n}, DataType::FLOAT64, AllocStrategy::DEVICE);
    auto B = engine.create_tensor({n, n}, DataType::FLOAT64, AllocStrategy::DEVICE);
    auto C = engine.create_tensor({n, n}, DataType::FLOAT64, AllocStrategy::DEVICE);
    std::vector<double> a(n * n), id(n * n, 0.0), c(n * n);
    for (int i = 0; i < n * n; ++i) a[i] = 0.5 * (i % 17) - 3.0;
    for (int i = 0; i < n; ++i) id[i * n + i] = 3.0;
    A.storage->copy_from_host(a.data(), a.size() * sizeof(double));
    B.storage->copy_from_host(id.data(), id.size() * sizeof(double));
    engine.blas().gemm(A, B, C);
    engine.execute().wait();
    C.storage->copy_to_host(c.data(), c.size() * sizeof(double));
    for (int i = 0; i < n * n; ++i) CHECK(c[i] == 3.0 * a[i]);
}

TEST_CASE(HostStrategyPinnedMapped, true)
{
    sb::Engine engine(ctx());
    auto A = engine.create_tensor({2, 2}, AllocStrategy::HOST);
    auto B = engine.create_tensor({2, 2}, AllocStrategy::HOST);
    auto C = engine.create_tensor({2, 2}, AllocStrategy::HOST);
    fill_tensor(A, {1, 2, 3, 4});
    fill_tensor(B, {0, 1, 1, 0});
    engine.blas().gemm(A, B, C);
    engine.execute().wait();
    verify_tensor(C, {2, 1, 4, 3});
}

TEST_CASE(FrameworkSimDeepForwardPass, true)  // test_framework_sim.cpp:10-73
{
    sb::Engine engine(ctx());
    const int batch_size = 512, features = 1024, num_layers = 10;
    auto X = engine.create_tensor({batch_size, features});
    fill_tensor(X, std::vector<float>(batch_size * features, 1.0f));
    std::vector<sb::Tensor> weights, activations{X};
    for (int i = 0; i < num_layers; ++i)
    {
        auto W = engine.create_tensor({features, features});
        fill_tensor(W, std::vector<float>(features * features, 0.01f));
        weights.push_back(W);
        activations.push_back(engine.create_tensor({batch_size, features}));
    }
    std::vector<std::string> names;
    engine.get_graph().set_trace_hook([&](const sr::Graph::TaskMetadata& m) { names.push_back(m.name); });
    // as the reference records it: a ReLU after every layer but the last
    // (the identity on these positive values)
    for (int i = 0; i < num_layers; ++i)
    {
        engine.blas().gemm(activations[i], weights[i], activations[i + 1]);
        if (i < num_layers - 1) engine.nonlinear().relu(activations[i + 1]);
    }
    engine.execute().wait();
    CHECK(activations.back().shape[0] == batch_size && activations.back().shape[1] == features);
    // each GEMM+ReLU pair ran as one fused task
    CHECK(names.size() == size_t(num_layers));
    for (int i = 0; i < num_layers - 1; ++i) CHECK(names[i] == "blas.lvl3.gemm+relu");
    CHECK(names.back() == "blas.lvl3.gemm");
    for (int l = 1; l <= num_layers; ++l)
    {
        const double expect = std::pow(1024.0 * double(0.01f), l);
        const float* p = activations[l].data_as<float>();
        for (int i = 0; i < batch_size * features; i += 4099)
            CHECK(std::fabs(p[i] - expect) <= 6.2e-5 * l * expect);
    }
}

TEST_CASE(FrameworkSimParallelBatchedInference, true)  // test_framework_sim.cpp:75-128
{
    sb::Engine engine(ctx());
    const int num_models = 24, m = 256, n = 512, k = 256;
    std::vector<sb::Tensor> inputs, weights, outputs;
    for (int i = 0; i < num_models; ++i)
    {
        auto X = engine.create_tensor({m, k});
        fill_tensor(X, std::vector<float>(m * k, 1.0f));
        inputs.push_back(X);
        auto W = engine.create_tensor({k, n});
        fill_tensor(W, std::vector<float>(k * n, 2.0f));
        weights.push_back(W);
        outputs.push_back(engine.create_tensor({m, n}));
    }
    std::vector<std::string> names;
    engine.get_graph().set_trace_hook([&](const sr::Graph::TaskMetadata& m) { names.push_back(m.name); });
    for (int i = 0; i < num_models; ++i)
    {
        engine.blas().gemm(inputs[i], weights[i], outputs[i]);
        engine.nonlinear().relu(outputs[i]);
    }
    engine.execute().wait();
    // every GEMM+ReLU pair fused; the 24 fused tasks go out as one grouped launch
    CHECK(names.size() == size_t(num_models));
    for (const auto& nm : names) CHECK(nm == "blas.lvl3.gemm+relu");
    for (int i = 0; i < num_models; ++i)
    {
        CHECK(outputs[i].shape[0] == m && outputs[i].shape[1] == n);
        verify_tensor(outputs[i], std::vector<float>(m * n, 512.0f), 0.0);
    }
}

TEST_CASE(DependencyManyReadersOneWriter, true)  // test_dependency_stress.cpp:9-57
{
    sb::Engine engine(ctx());
    const int num_readers = 5000, N = 32;
    auto writer = engine.create_tensor({N, N});
    fill_tensor(writer, std::vector<float>(N * N, 1.0f));
    std::vector<sb::Tensor> outs;
    for (int i = 0; i < num_readers; ++i)
    {
        auto t = engine.create_tensor({N, N});
        fill_tensor(t, std::vector<float>(N * N, 0.0f));
        outs.push_back(t);
    }
    auto w = engine.create_tensor({N, N});
    fill_tensor(w, std::vector<float>(N * N, 2.0f));
    engine.blas().gemm(w, w, writer);                   // writer = 2*2*32 = 128
    for (int i = 0; i < num_readers; ++i) engine.blas().gemm(writer, w, outs[i]);  // 128*2*32
    engine.execute().wait();
    verify_tensor(writer, std::vector<float>(N * N, 128.0f), 0.0);
    for (int i = 0; i < num_readers; i += 499) verify_tensor(outs[i], std::vector<float>(N * N, 8192.0f), 0.0);
    verify_tensor(outs.back(), std::vector<float>(N * N, 8192.0f), 0.0);
}

TEST_CASE(DependencyShardCollision, true)  // test_dependency_stress.cpp:59-95
{
    sb::Engine engine(ctx());
    const int num_ops = 3000, N = 8;
    std::vector<sb::Tensor> As, Bs, Cs;
    for (int i = 0; i < num_ops; ++i)
    {
        As.push_back(engine.create_tensor({N, N}));
        Bs.push_back(engine.create_tensor({N, N}));
        Cs.push_back(engine.create_tensor({N, N}));
        fill_tensor(As.back(), std::vector<float>(N * N, float(i % 7)));
        fill_tensor(Bs.back(), std::vector<float>(N * N, 1.0f));
    }
    for (int i = 0; i < num_ops; ++i) engine.blas().gemm(As[i], Bs[i], Cs[i]);
    engine.execute().wait();
    for (int i = 0; i < num_ops; i += 97) verify_tensor(Cs[i], std::vector<float>(N * N, 8.0f * (i % 7)), 0.0);
}

TEST_CASE(TraceHookSeesGemmMetadata, true)
{
    sb::Engine engine(ctx());
    std::vector<std::string> names;
    float alpha_seen = 0;
    engine.get_graph().set_trace_hook([&](const sr::Graph::TaskMetadata& m) {
        names.push_back(m.name);
        alpha_seen = m.get_param<float>(0);
    });
    auto A = engine.create_tensor({4, 4});
    auto B = engine.create_tensor({4, 4});
    auto C = engine.create_tensor({4, 4});
    fill_tensor(A, std::vector<float>(16, 1.0f));
    fill_tensor(B, std::vector<float>(16, 1.0f));
    engine.blas().gemm(A, B, C, false, false, 0.5f, 0.0f);
    engine.execute().wait();
    CHECK(names.size() == 1 && names[0] == "blas.lvl3.gemm" && alpha_seen == 0.5f);
    verify_tensor(C, std::vector<float>(16, 2.0f), 0.0);
}

TEST_CASE(ReluRejectsUnsupportedTypes, false)
{
    sr::Execution::RuntimeContext local;
    sb::Engine e(local);
    sb::Tensor h(nullptr, {4, 4}), z(nullptr, {4, 4}), f(nullptr, {4, 4});
    h.dtype = DataType::HALF;
    z.dtype = DataType::COMPLEX64;
    CHECK_THROWS(e.nonlinear().relu(h));
    CHECK_THROWS(e.nonlinear().relu(z));
    CHECK_THROWS(e.nonlinear().relu(f));  // no storage
    CHECK(e.get_graph().pending() == 0);
}

namespace
{
    template <typename T>
    void relu_special_values(DataType dt)
    {
        // relu.cpp:38-41: x > 0 ? x : 0, so NaN and -0 become +0
        sb::Engine engine(ctx());
        const T inf = std::numeric_limits<T>::infinity(), nan = std::numeric_limits<T>::quiet_NaN();
        const T tiny = std::numeric_limits<T>::denorm_min();
        std::vector<T> in = {T(-1.5), T(0), T(-0.0), T(2.25), nan, -nan, inf, -inf, tiny, -tiny, T(1e30), T(-1e30)};
        std::vector<T> want = {0, 0, 0, T(2.25), 0, 0, inf, 0, tiny, 0, T(1e30), 0};
        // a length that is not a multiple of the kernel's vector width
        const int n = 1000 * int(in.size()) + 5;
        auto t = engine.create_tensor({n}, dt);
        std::vector<T> data(n), expect(n);
        for (int i = 0; i < n; ++i)
        {
            data[i] = in[i % in.size()] * (i < int(in.size()) ? T(1) : T(1 + (i % 3)));
            expect[i] = data[i] > T(0) ? data[i] : T(0);
        }
        for (size_t i = 0; i < in.size(); ++i) CHECK(std::memcmp(&expect[i], &want[i], sizeof(T)) == 0 || expect[i] == want[i]);
        fill_tensor<T>(t, data);
        engine.nonlinear().relu(t);
        engine.execute().wait();
        const T* got = t.data_as<T>();
        for (int i = 0; i < n; ++i) CHECK(std::memcmp(&got[i], &expect[i], sizeof(T)) == 0);
    }
} // namespace

TEST_CASE(ReluSpecialValuesFp32AndFp64, true)
{
    relu_special_values<float>(DataType::FLOAT32);
    relu_special_values<double>(DataType::FLOAT64);
}

TEST_CASE(ReluOnRowSliceTouchesOnlyTheSlice, true)
{
    sb::Engine engine(ctx());
    auto X = engine.create_tensor({4, 8});
    std::vector<float> x(32);
    for (int i = 0; i < 32; ++i) x[i] = (i % 2) ? -1.0f * i : 1.0f * i;
    fill_tensor(X, x);
    auto rows = X.slice(0, 1, 3);  // rows 1 and 2
    engine.nonlinear().relu(rows);
    engine.execute().wait();
    const float* p = X.data_as<float>();
    for (int i = 0; i < 32; ++i)
    {
        const bool inside = i >= 8 && i < 24;
        CHECK(p[i] == (inside ? (x[i] > 0 ? x[i] : 0.0f) : x[i]));
    }
}

namespace
{
    // C = relu(alpha*A*B + beta*C) through the engine, fused or not.
    template <typename T>
    std::vector<T> gemm_relu_via_engine(DataType dt, bool fuse, int batch, std::vector<std::string>& names)
    {
        sb::Engine engine(ctx());
        engine.get_graph().set_fusion(fuse);
        engine.get_graph().set_trace_hook([&](const sr::Graph::TaskMetadata& m) { names.push_back(m.name); });
        const int m = 130, n = 97, k = 75;
        auto A = batch > 1 ? engine.create_tensor({batch, m, k}, dt) : engine.create_tensor({m, k}, dt);
        auto B = batch > 1 ? engine.create_tensor({batch, k, n}, dt) : engine.create_tensor({k, n}, dt);
        auto C = batch > 1 ? engine.create_tensor({batch, m, n}, dt) : engine.create_tensor({m, n}, dt);
        std::vector<T> a(A.num_elements), b(B.num_elements), c(C.num_elements);
        for (size_t i = 0; i < a.size(); ++i) a[i] = T(std::sin(0.7 * i));
        for (size_t i = 0; i < b.size(); ++i) b[i] = T(std::cos(0.3 * i));
        for (size_t i = 0; i < c.size(); ++i) c[i] = T(0.5 * ((i % 11) - 5));
        fill_tensor<T>(A, a);
        fill_tensor<T>(B, b);
        fill_tensor<T>(C, c);
        engine.blas().gemm(A, B, C, false, false, 0.75f, 0.5f);
        engine.nonlinear().relu(C);
        engine.execute().wait();
        const T* p = C.data_as<T>();
        std::vector<T> out(p, p + C.num_elements);
        // against a double host loop
        double num = 0, den = 0;
        for (int q = 0; q < batch; ++q)
            for (int i = 0; i < m; ++i)
                for (int j = 0; j < n; ++j)
                {
                    double s = 0;
                    for (int l = 0; l < k; ++l) s += double(a[(q * m + i) * k + l]) * double(b[(q * k + l) * n + j]);
                    double want = 0.75 * s + 0.5 * double(c[(q * m + i) * n + j]);
                    want = want > 0 ? want : 0;
                    const double g = out[(q * m + i) * n + j];
                    CHECK(g >= 0);
                    num += (g - want) * (g - want);
                    den += want * want;
                }
        CHECK(std::sqrt(num / den) <= (sizeof(T) == 4 ? 1e-5 : 1e-12));
        return out;
    }
} // namespace

TEST_CASE(GemmReluFusedEqualsUnfused, true)
{
    for (int batch : {1, 3})
    {
        std::vector<std::string> fused_names, plain_names;
        auto f32a = gemm_relu_via_engine<float>(DataType::FLOAT32, true, batch, fused_names);
        auto f32b = gemm_relu_via_engine<float>(DataType::FLOAT32, false, batch, plain_names);
        CHECK(fused_names.size() == 1 && fused_names[0] == "blas.lvl3.gemm+relu");
        CHECK(plain_names.size() == 2 && plain_names[0] == "blas.lvl3.gemm" &&
              plain_names[1] == "math.nonlinear.relu");
        // same GEMM kernel, same values: the fused epilogue is bit-identical
        CHECK(std::memcmp(f32a.data(), f32b.data(), f32a.size() * sizeof(float)) == 0);
        fused_names.clear();
        plain_names.clear();
        auto f64a = gemm_relu_via_engine<double>(DataType::FLOAT64, true, batch, fused_names);
        auto f64b = gemm_relu_via_engine<double>(DataType::FLOAT64, false, batch, plain_names);
        CHECK(fused_names.size() == 1 && plain_names.size() == 2);
        CHECK(std::memcmp(f64a.data(), f64b.data(), f64a.size() * sizeof(double)) == 0);
    }
}

TEST_CASE(ReluNotFusedUnlessSameRegion, true)
{
    sb::Engine engine(ctx());
    std::vector<std::string> names;
    engine.get_graph().set_trace_hook([&](const sr::Graph::TaskMetadata& m) { names.push_back(m.name); });
    auto A = engine.create_tensor({8, 8});
    auto B = engine.create_tensor({8, 8});
    auto C = engine.create_tensor({8, 8});
    auto D = engine.create_tensor({8, 8});
    std::vector<float> a(64), b(64, 1.0f), d(64);
    for (int i = 0; i < 64; ++i) a[i] = ((i / 8) % 2) ? -1.0f : 1.0f;   // C rows alternate +-8
    for (int i = 0; i < 64; ++i) d[i] = (i % 3) ? -2.0f : 3.0f;
    fill_tensor(A, a);
    fill_tensor(B, b);
    fill_tensor(D, d);
    // 1. ReLU on another tensor right after the GEMM: not fused
    engine.blas().gemm(A, B, C);
    engine.nonlinear().relu(D);
    // 2. ReLU on part of the GEMM output: not fused
    auto C2 = engine.create_tensor({8, 8});
    engine.blas().gemm(A, B, C2);
    auto top = C2.slice(0, 0, 4);
    engine.nonlinear().relu(top);
    // 3. GEMM into a row slice, ReLU over exactly that slice: fused
    auto C3 = engine.create_tensor({8, 8});
    fill_tensor(C3, std::vector<float>(64, -5.0f));
    auto mid = C3.slice(0, 2, 6);
    auto A4 = engine.create_tensor({4, 8});
    fill_tensor(A4, std::vector<float>(a.begin(), a.begin() + 32));
    engine.blas().gemm(A4, B, mid);
    engine.nonlinear().relu(mid);
    engine.execute().wait();
    CHECK(names.size() == 5);
    CHECK(names[0] == "blas.lvl3.gemm" && names[1] == "math.nonlinear.relu");
    CHECK(names[2] == "blas.lvl3.gemm" && names[3] == "math.nonlinear.relu");
    CHECK(names[4] == "blas.lvl3.gemm+relu");
    // values: C untouched by ReLU, D rectified, C2 top half rectified,
    // C3 rows 2..5 rectified GEMM rows, the rest still -5
    const float* c = C.data_as<float>();
    const float* dd = D.data_as<float>();
    const float* c2 = C2.data_as<float>();
    const float* c3 = C3.data_as<float>();
    for (int i = 0; i < 64; ++i)
    {
        const float row = (i / 8 % 2) ? -8.0f : 8.0f;
        CHECK(c[i] == row);
        CHECK(dd[i] == (d[i] > 0 ? d[i] : 0.0f));
        CHECK(c2[i] == (i < 32 ? (row > 0 ? row : 0.0f) : row));
        const int r = i / 8;
        CHECK(c3[i] == ((r >= 2 && r < 6) ? ((r % 2) ? 0.0f : 8.0f) : -5.0f));
    }
}

// ------------------------------------------------------------- GEMV / SYRK

TEST_CASE(GemvSyrkValidationThrowsAtRecordTime, false)
{
    sr::Execution::RuntimeContext local;
    sb::Engine e(local);
    sb::Tensor A(nullptr, {2, 3}), x3(nullptr, {3}), y2(nullptr, {2}), v1(nullptr, {3});
    sb::Tensor m23(nullptr, {2, 3}), y3(nullptr, {3});
    CHECK_THROWS(e.blas().gemv(v1, x3, y2));             // rank < 2 (gemv.cpp:68)
    CHECK_THROWS(e.blas().gemv(A, y2, y2));              // x length != n (gemv.cpp:88)
    CHECK_THROWS(e.blas().gemv(A, x3, y3));              // y length != m (gemv.cpp:89)
    CHECK_THROWS(e.blas().gemv(A, x3, y3, true));        // transposed: x needs m
    sb::Tensor xd(nullptr, {3});
    xd.dtype = DataType::FLOAT64;
    CHECK_THROWS(e.blas().gemv(A, xd, y2));              // dtype mismatch
    sb::Tensor xs(nullptr, {3, 1});
    xs = xs.transpose(0, 1);                             // non-contiguous rank 2 vector
    CHECK_THROWS(e.blas().gemv(A, xs, y2));
    sb::Tensor Az(nullptr, {2, 3}), xz(nullptr, {3}), yz(nullptr, {2});
    Az.dtype = xz.dtype = yz.dtype = DataType::COMPLEX32;
    CHECK_THROWS(e.blas().gemv(Az, xz, yz));             // not provided
    sb::Tensor S(nullptr, {3, 2}), Cr(nullptr, {3, 4}), Cs(nullptr, {3, 3}), C2(nullptr, {2, 2});
    CHECK_THROWS(e.blas().syrk(v1, Cs));                 // rank < 2
    CHECK_THROWS(e.blas().syrk(S, Cr));                  // C not square (syrk.cpp:96)
    CHECK_THROWS(e.blas().syrk(S, C2));                  // A rows != n (syrk.cpp:102)
    CHECK_THROWS(e.blas().syrk(S, Cs, false, true));     // A^T has 2 rows != 3
    sb::Tensor Sh(nullptr, {3, 2}), Ch(nullptr, {3, 3});
    Sh.dtype = Ch.dtype = DataType::HALF;
    CHECK_THROWS(e.blas().syrk(Sh, Ch));
    CHECK(e.get_graph().pending() == 0);
}

TEST_CASE(GroupPlannerRunsAndTableOffsets, false)
{
    // host-only: runs break at key/epilogue changes, explicit deps and hazards;
    // every run's table slice holds exactly its members' pointers, in order
    struct Fake
    {
        sr::Graph::GroupHook g;
        std::vector<void*> r, w;
        bool deps = false;
    };
    std::vector<Fake> f(12);
    char mem[64][16];
    auto P = [&](int i) { return static_cast<void*>(mem[i]); };
    for (int i = 0; i < 12; ++i)
    {
        f[i].g.enabled = true;
        f[i].g.key[1] = 8;
        f[i].g.ptrs[0] = P(3 * i);
        f[i].g.ptrs[1] = P(3 * i + 1);
        f[i].g.ptrs[2] = P(3 * i + 2);
        f[i].g.aligned = (i % 5) != 4;
        f[i].g.launch = [](sr::Execution::Queue&, const void* const*, int64_t, bool, int) {};
        f[i].r = {P(3 * i), P(3 * i + 1)};
        f[i].w = {P(3 * i + 2)};
    }
    f[3].g.key[1] = 9;                 // breaks the run 0..2
    f[6].g.epilogue = 1;               // breaks 4..5
    f[8].r[0] = f[7].w[0];             // RAW on 7: breaks 6? no: 6 has another epilogue; 7..8 broken
    f[10].deps = true;                 // not groupable
    std::vector<sr::Graph::GroupCandidate> c(12);
    for (int i = 0; i < 12; ++i) c[i] = sr::Graph::GroupCandidate{&f[i].g, f[i].deps, &f[i].r, &f[i].w};
    std::vector<const void*> table;
    const auto runs = sr::Graph::plan_groups(c, table);
    // expected runs: [0,3), [4,6), [8,10) (8 starts a new run after the hazard), none after
    CHECK(runs.size() == 3);
    const size_t firsts[] = {0, 4, 8}, counts[] = {3, 2, 2};
    int64_t off = 0;
    for (size_t k = 0; k < runs.size(); ++k)
    {
        CHECK(runs[k].first == firsts[k] && runs[k].count == counts[k]);
        CHECK(runs[k].table_offset == off);
        bool aligned = true;
        for (size_t q = 0; q < runs[k].count; ++q)
        {
            const auto& g = f[runs[k].first + q].g;
            for (int e = 0; e < 3; ++e) CHECK(table[3 * (runs[k].table_offset + q) + e] == g.ptrs[e]);
            aligned = aligned && g.aligned;
        }
        CHECK(runs[k].aligned == aligned);
        off += static_cast<int64_t>(runs[k].count);
    }
    CHECK(table.size() == size_t(3 * off));
    // a WAR inside a run: task 1 writes what task 0 reads
    std::vector<Fake> h(2);
    for (int i = 0; i < 2; ++i)
    {
        h[i].g = f[0].g;
        h[i].w = {P(40 + i)};
    }
    h[0].r = {P(50)};
    h[1].r = {P(51)};
    h[1].w = {P(50)};
    std::vector<sr::Graph::GroupCandidate> c2 = {{&h[0].g, false, &h[0].r, &h[0].w},
                                                 {&h[1].g, false, &h[1].r, &h[1].w}};
    CHECK(sr::Graph::plan_groups(c2, table).empty() && table.empty());
}

TEST_CASE(SimpleGEMV, true)  // tests/blas/level2/test_gemv.cpp
{
    sb::Engine engine(ctx());
    auto A = engine.create_tensor({2, 3});
    auto X = engine.create_tensor({3});
    auto Y = engine.create_tensor({2});
    fill_tensor(A, {1, 2, 3, 4, 5, 6});
    fill_tensor(X, {1, 1, 1});
    fill_tensor(Y, {0, 0});
    engine.blas().gemv(A, X, Y);
    engine.execute().wait();
    verify_tensor(Y, {6, 15}, 0.0);
}

TEST_CASE(SimpleSYRK, true)  // tests/blas/level3/test_syrk.cpp
{
    sb::Engine engine(ctx());
    auto A = engine.create_tensor({3, 2});
    auto C = engine.create_tensor({3, 3});
    fill_tensor(A, {1, 2, 3, 4, 5, 6});
    fill_tensor(C, std::vector<float>(9, 0.0f));
    engine.blas().syrk(A, C, false, false, 1.0f, 0.0f);
    engine.execute().wait();
    verify_tensor(C, {5, 0, 0, 11, 25, 0, 17, 39, 61}, 0.0);
}

TEST_CASE(SimpleSYRKColumnMajor, true)  // tests/blas/level3/test_syrk.cpp
{
    sb::Engine engine(ctx(), Layout::COLUMN_MAJOR);
    auto A = engine.create_tensor({3, 2});  // transA: A is K x N
    auto C = engine.create_tensor({2, 2});
    fill_tensor(A, {1, 2, 3, 4, 5, 6});
    fill_tensor(C, std::vector<float>(4, 0.0f));
    engine.blas().syrk(A, C, false, true, 1.0f, 0.0f);
    engine.execute().wait();
    verify_tensor(C, {14, 32, 0, 77}, 0.0);
}

TEST_CASE(GemvTransposedStridedFp64, true)
{
    // y (n) = 0.5 * A^T x + 2 y with x a rank-1 view of stride 3, fp64
    sb::Engine engine(ctx());
    const int m = 37, n = 29;
    auto A = engine.create_tensor({m, n}, DataType::FLOAT64);
    auto Xbuf = engine.create_tensor({3 * m}, DataType::FLOAT64);
    auto Y = engine.create_tensor({n}, DataType::FLOAT64);
    std::vector<double> a(m * n), xb(3 * m), y(n);
    for (int i = 0; i < m * n; ++i) a[i] = std::sin(0.1 * i);
    for (int i = 0; i < 3 * m; ++i) xb[i] = std::cos(0.2 * i);
    for (int i = 0; i < n; ++i) y[i] = 0.125 * i;
    fill_tensor<double>(A, a);
    fill_tensor<double>(Xbuf, xb);
    fill_tensor<double>(Y, y);
    sb::Tensor X = Xbuf;  // the view x[i] = xb[3 i]
    X.shape[0] = m;
    X.num_elements = m;
    X.strides[0] = 3;
    engine.blas().gemv(A, X, Y, true, 0.5f, 2.0f);
    engine.execute().wait();
    const double* got = Y.data_as<double>();
    for (int j = 0; j < n; ++j)
    {
        double s = 0;
        for (int i = 0; i < m; ++i) s += a[i * n + j] * xb[3 * i];
        CHECK_NEAR(got[j], 0.5 * s + 2.0 * y[j], 1e-13);
    }
}

TEST_CASE(SyrkBatchedUpperMatchesHostLoop, true)
{
    // rank-3: 3 problems of C (40x40) = A (40x17) A^T, upper triangle, beta = 1
    sb::Engine engine(ctx());
    const int b = 3, n = 40, k = 17;
    auto A = engine.create_tensor({b, n, k});
    auto C = engine.create_tensor({b, n, n});
    std::vector<float> a(b * n * k), c(b * n * n);
    for (size_t i = 0; i < a.size(); ++i) a[i] = std::sin(0.3f * i);
    for (size_t i = 0; i < c.size(); ++i) c[i] = 0.5f * ((i % 7) - 3);
    fill_tensor(A, a);
    fill_tensor(C, c);
    std::vector<std::string> names;
    engine.get_graph().set_trace_hook([&](const sr::Graph::TaskMetadata& m) { names.push_back(m.name); });
    engine.blas().syrk(A, C, true, false, 1.0f, 1.0f);
    engine.execute().wait();
    CHECK(names.size() == 1 && names[0] == "blas.lvl3.syrk");
    const float* got = C.data_as<float>();
    for (int q = 0; q < b; ++q)
        for (int i = 0; i < n; ++i)
            for (int j = 0; j < n; ++j)
            {
                const int idx = q * n * n + i * n + j;
                if (j < i)
                {
                    CHECK(got[idx] == c[idx]);  // lower triangle untouched
                    continue;
                }
                double s = 0;
                for (int l = 0; l < k; ++l) s += double(a[(q * n + i) * k + l]) * a[(q * n + j) * k + l];
                CHECK_NEAR(got[idx], s + c[idx], 1e-4);
            }
}

// -------------------------------------------------------------------- .npy IO

namespace
{
    std::string npy_dir()
    {
        const char* d = std::getenv("SBX_NPY_DIR");
        if (!d || !*d) throw Skip{"SBX_NPY_DIR not set"};
        return d;
    }

    std::string tmp_path(const std::string& name)
    {
        const char* t = std::getenv("TMPDIR");
        return std::string(t && *t ? t : "/tmp") + "/sbx_io_" + std::to_string(getpid()) + "_" + name;
    }

    std::string file_bytes(const std::string& path, size_t max_bytes = size_t(-1))
    {
        std::ifstream f(path, std::ios::binary);
        CHECK(f.good());
        std::string s((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
        return s.substr(0, std::min(max_bytes, s.size()));
    }

    // host image of a tensor's elements (contiguous tensors)
    std::vector<char> host_bytes(const sb::Tensor& t)
    {
        const size_t n = size_t(t.num_elements) * sb::IO::element_bytes(t.dtype);
        std::vector<char> out(n);
        if (t.storage->strategy == AllocStrategy::DEVICE)
            t.storage->copy_to_host(out.data(), n, t.offset_bytes());
        else
            std::memcpy(out.data(), t.data(), n);
        return out;
    }

    void set_host_bytes(sb::Tensor& t, const std::vector<char>& in)
    {
        if (t.storage->strategy == AllocStrategy::DEVICE)
            t.storage->copy_from_host(in.data(), in.size(), t.offset_bytes());
        else
            std::memcpy(t.data(), in.data(), in.size());
    }
} // namespace

TEST_CASE(NpyHeaderEncodeAndParse, false)  // src/io.cpp:136-180
{
    const int64_t s23[] = {2, 3};
    const std::string h = sb::IO::npy_header(DataType::FLOAT32, Layout::ROW_MAJOR, s23, 2);
    const std::string dict = "{'descr': '<f4', 'fortran_order': False, 'shape': (2, 3), }";
    CHECK(h.size() == 128);
    CHECK(h.compare(0, 8, std::string("\x93NUMPY\x01\x00", 8)) == 0);
    CHECK(static_cast<unsigned char>(h[8]) == 118 && h[9] == 0);  // 128 - 10
    CHECK(h.compare(10, dict.size(), dict) == 0);
    CHECK(h.back() == '\n' && h[10 + dict.size()] == ' ');
    const int64_t s5[] = {5};
    const std::string h1 = sb::IO::npy_header(DataType::FLOAT64, Layout::COLUMN_MAJOR, s5, 1);
    CHECK(h1.find("{'descr': '<f8', 'fortran_order': True, 'shape': (5,), }") == 10);
    CHECK(h1.size() % 64 == 0);
    for (const std::string& pre : {h, h1})
    {
        const sb::NpyHeader p = sb::IO::parse_npy_header(pre);
        CHECK(p.data_offset == pre.size());
    }
    const sb::NpyHeader p = sb::IO::parse_npy_header(h);
    CHECK(p.descr == "<f4" && !p.fortran_order && p.shape.size() == 2 && p.shape[0] == 2 &&
          p.shape[1] == 3);
    const sb::NpyHeader p1 = sb::IO::parse_npy_header(h1);
    CHECK(p1.descr == "<f8" && p1.fortran_order && p1.shape.size() == 1 && p1.shape[0] == 5);
    // version 2.0 (4-byte length), other key order and spacing, rank 0
    std::string d2 = "{\"shape\":(),\"fortran_order\":False,\"descr\":\"<c16\"}\n";
    std::string v2("\x93NUMPY\x02\x00", 8);
    for (int i = 0; i < 4; ++i) v2 += static_cast<char>((d2.size() >> (8 * i)) & 0xff);
    v2 += d2;
    const sb::NpyHeader q = sb::IO::parse_npy_header(v2);
    CHECK(q.descr == "<c16" && q.shape.empty() && q.data_offset == v2.size());
    // malformed
    CHECK_THROWS(sb::IO::parse_npy_header("\x93NUMPX\x01\x00\x00\x00"));
    std::string bad = h;
    bad[10 + dict.find("(2")] = '[';
    CHECK_THROWS(sb::IO::parse_npy_header(bad));
    CHECK_THROWS(sb::IO::parse_npy_header(h.substr(0, 40)));  // truncated
    CHECK(std::string(sb::IO::npy_descr(DataType::HALF)) == "<f2" &&
          std::string(sb::IO::npy_descr(DataType::COMPLEX32)) == "<c8" &&
          sb::IO::element_bytes(DataType::COMPLEX64) == 16);
}

TEST_CASE(NpyHeadersMatchNumpy, false)
{
    // headers.txt: "<file> <dtype> <layout> <rank> <d0> <d1> ..." for files np.save wrote
    const std::string dir = npy_dir();
    std::ifstream list(dir + "/headers.txt");
    CHECK(list.good());
    int n = 0;
    std::string file;
    int dtype, layout, rank;
    while (list >> file >> dtype >> layout >> rank)
    {
        int64_t dims[sb::Core::MAX_TENSOR_RANK] = {0};
        for (int i = 0; i < rank; ++i) list >> dims[i];
        const std::string want = sb::IO::npy_header(static_cast<DataType>(dtype),
                                                    static_cast<Layout>(layout), dims, rank);
        const std::string got = file_bytes(dir + "/" + file, want.size());
        if (got != want) throw Failure{"header of " + file + " differs from numpy's"};
        const sb::NpyHeader p = sb::IO::parse_npy_header(file_bytes(dir + "/" + file, 4096));
        CHECK(static_cast<int>(p.shape.size()) == rank && p.data_offset == want.size());
        ++n;
    }
    CHECK(n > 0);
}

TEST_CASE(NpyRoundTripEveryStrategyAndType, true)
{
    sb::Engine engine(ctx());
    const DataType types[] = {DataType::FLOAT32, DataType::FLOAT64, DataType::HALF,
                              DataType::COMPLEX32, DataType::COMPLEX64};
    const AllocStrategy strats[] = {AllocStrategy::DEVICE, AllocStrategy::SHARED, AllocStrategy::HOST};
    int which = 0;
    for (AllocStrategy st : strats)
        for (DataType dt : types)
        {
            // create_tensor(HALF) cannot hold 37 x 53: the Tensor constructor checks
            // capacity at 4 bytes per element (tensor.hpp:123 of the reference), so
            // HALF tensors get storage sized that way
            auto make = [&]() {
                if (dt != DataType::HALF) return engine.create_tensor({37, 53}, dt, st);
                auto storage = sr::make_sushi<sb::Storage>(ctx().get_allocator(), 37 * 53 * 4, st);
                sb::Tensor h(storage, {37, 53});
                h.dtype = DataType::HALF;
                return h;
            };
            auto t = make();
            std::vector<char> img(size_t(t.num_elements) * sb::IO::element_bytes(dt));
            for (size_t i = 0; i < img.size(); ++i) img[i] = char((i * 131 + which * 7) & 0xff);
            set_host_bytes(t, img);
            const std::string path = tmp_path("rt" + std::to_string(which++) + ".npy");
            engine.io().save_npy(t, path);
            const std::string pre = sb::IO::npy_header(dt, Layout::ROW_MAJOR, t.shape.data(), 2);
            const std::string bytes = file_bytes(path);
            CHECK(bytes.size() == pre.size() + img.size());
            CHECK(bytes.compare(0, pre.size(), pre) == 0);
            CHECK(std::memcmp(bytes.data() + pre.size(), img.data(), img.size()) == 0);
            auto u = make();
            engine.io().load_npy(u, path);
            CHECK(host_bytes(u) == img);
            // raw binary dump of the same elements
            const std::string bin = tmp_path("rt.bin");
            engine.io().save_bin(t, bin);
            CHECK(file_bytes(bin) == std::string(img.begin(), img.end()));
            auto w = make();
            engine.io().load_bin(w, bin);
            CHECK(host_bytes(w) == img);
            std::remove(path.c_str());
            std::remove(bin.c_str());
        }
}

TEST_CASE(NpyViewsOrdersAndErrors, true)
{
    // a transposed (non-contiguous) view is written in its logical order
    sb::Engine engine(ctx());
    auto X = engine.create_tensor({4, 6}, DataType::FLOAT32, AllocStrategy::DEVICE);
    std::vector<float> x(24);
    for (int i = 0; i < 24; ++i) x[i] = float(i) + 0.5f;
    X.storage->copy_from_host(x.data(), x.size() * 4);
    auto XT = X.transpose(0, 1);  // 6 x 4 view
    const std::string p1 = tmp_path("view.npy");
    engine.io().save_npy(XT, p1);
    auto Y = engine.create_tensor({6, 4}, DataType::FLOAT32, AllocStrategy::SHARED);
    engine.io().load_npy(Y, p1);
    const float* y = Y.data_as<float>();
    for (int i = 0; i < 6; ++i)
        for (int j = 0; j < 4; ++j) CHECK(y[i * 4 + j] == x[j * 6 + i]);
    // reading into a transposed view scatters by strides
    auto Z = engine.create_tensor({4, 6}, DataType::FLOAT32, AllocStrategy::DEVICE);
    auto ZT = Z.transpose(0, 1);
    engine.io().load_npy(ZT, p1);
    std::vector<float> z(24);
    Z.storage->copy_to_host(z.data(), 96);
    CHECK(z == x);
    // a C-order file read into a column-major tensor is reordered
    sb::Engine colmajor(ctx(), Layout::COLUMN_MAJOR);
    auto C = colmajor.create_tensor({6, 4}, DataType::FLOAT32, AllocStrategy::HOST);
    colmajor.io().load_npy(C, p1);
    const float* c = C.data_as<float>();
    for (int i = 0; i < 6; ++i)
        for (int j = 0; j < 4; ++j) CHECK(c[i + 6 * j] == x[j * 6 + i]);
    // and written back with fortran_order True, in column-major order
    const std::string p2 = tmp_path("colmajor.npy");
    colmajor.io().save_npy(C, p2);
    const sb::NpyHeader h = sb::IO::parse_npy_header(file_bytes(p2, 4096));
    CHECK(h.fortran_order && h.shape.size() == 2 && h.shape[0] == 6 && h.shape[1] == 4);
    // errors: wrong dtype, wrong shape, wrong rank, truncated, bad magic, missing file
    auto D = engine.create_tensor({6, 4}, DataType::FLOAT64, AllocStrategy::SHARED);
    CHECK_THROWS(engine.io().load_npy(D, p1));
    auto E = engine.create_tensor({4, 6}, DataType::FLOAT32, AllocStrategy::SHARED);
    CHECK_THROWS(engine.io().load_npy(E, p1));
    auto F = engine.create_tensor({24}, DataType::FLOAT32, AllocStrategy::SHARED);
    CHECK_THROWS(engine.io().load_npy(F, p1));
    const std::string full = file_bytes(p1);
    const std::string p3 = tmp_path("short.npy");
    {
        std::ofstream o(p3, std::ios::binary);
        o << full.substr(0, full.size() - 8);
    }
    CHECK_THROWS(engine.io().load_npy(Y, p3));
    {
        std::ofstream o(p3, std::ios::binary);
        o << "NOTNUMPY" << full.substr(8);
    }
    CHECK_THROWS(engine.io().load_npy(Y, p3));
    CHECK_THROWS(engine.io().load_npy(Y, tmp_path("missing.npy")));
    for (const auto& p : {p1, p2, p3}) std::remove(p.c_str());
}

TEST_CASE(NpyLargeDeviceTensorStreams, true)
{
    // 3 x 100 MB chunks through the pinned double buffer, both directions
    sb::Engine engine(ctx());
    const int64_t n = (int64_t(75) << 20) + 17;  // 300 MB + 68 B of fp32
    auto T = engine.create_tensor({n}, DataType::FLOAT32, AllocStrategy::DEVICE);
    std::vector<float> v(n);
    for (int64_t i = 0; i < n; ++i) v[i] = float(i % 1000003) * 0.25f;
    T.storage->copy_from_host(v.data(), size_t(n) * 4);
    const std::string p = tmp_path("large.npy");
    engine.io().save_npy(T, p);
    auto U = engine.create_tensor({n}, DataType::FLOAT32, AllocStrategy::DEVICE);
    engine.io().load_npy(U, p);
    std::vector<float> w(n);
    U.storage->copy_to_host(w.data(), size_t(n) * 4);
    CHECK(std::memcmp(w.data(), v.data(), size_t(n) * 4) == 0);
    std::remove(p.c_str());
}

TEST_CASE(GoldenGemmThroughNpy, true)
{
    // cases.txt: "<name> <dtype> <layout> <ta> <tb> <m> <n> <k> <alpha> <beta>"; the
    // operands are <name>_{A,B,C,out}.npy written by numpy; the result goes to
    // <name>_got.npy through save_npy
    const std::string dir = npy_dir();
    std::ifstream list(dir + "/cases.txt");
    CHECK(list.good());
    std::string name;
    int dt, layout, ta, tb;
    int64_t m, n, k;
    double alpha, beta;
    int cases = 0;
    while (list >> name >> dt >> layout >> ta >> tb >> m >> n >> k >> alpha >> beta)
    {
        sb::Engine engine(ctx(), static_cast<Layout>(layout));
        const DataType dtype = static_cast<DataType>(dt);
        auto A = ta ? engine.create_tensor({k, m}, dtype) : engine.create_tensor({m, k}, dtype);
        auto B = tb ? engine.create_tensor({n, k}, dtype) : engine.create_tensor({k, n}, dtype);
        auto C = engine.create_tensor({m, n}, dtype);
        auto Want = engine.create_tensor({m, n}, dtype);
        engine.io().load_npy(A, dir + "/" + name + "_A.npy");
        engine.io().load_npy(B, dir + "/" + name + "_B.npy");
        engine.io().load_npy(C, dir + "/" + name + "_C.npy");
        engine.io().load_npy(Want, dir + "/" + name + "_out.npy");
        engine.blas().gemm(A, B, C, ta != 0, tb != 0, float(alpha), float(beta));
        engine.io().save_npy(C, dir + "/" + name + "_got.npy");  // runs the GEMM first
        double num = 0, den = 0;
        for (int64_t i = 0; i < m * n; ++i)
        {
            const double g = dtype == DataType::FLOAT32 ? C.data_as<float>()[i] : C.data_as<double>()[i];
            const double w = dtype == DataType::FLOAT32 ? Want.data_as<float>()[i]
                                                        : Want.data_as<double>()[i];
            num += (g - w) * (g - w);
            den += w * w;
        }
        const double err = den > 0 ? std::sqrt(num / den) : std::sqrt(num);
        if (err > (dtype == DataType::FLOAT32 ? 1e-5 : 1e-12))
            throw Failure{name + ": normwise error " + std::to_string(err)};
        ++cases;
    }
    CHECK(cases > 0);
}

// ------------------------------------------------------------ multi-lane DAG

namespace
{
    // Runs a seeded random DAG of GEMMs over `nbuf` shared 192x192 buffers
    // (dst = 0.01 * src1 * src2 + 0.5 * dst, with RAW/WAR/WAW hazards all
    // over) on `lanes` lanes; returns every buffer's bytes afterwards.
    std::vector<float> random_dag(size_t lanes, int nbuf, int nops, unsigned seed, bool grouping = true)
    {
        sb::Engine engine(ctx());
        engine.get_graph().set_max_lanes(lanes);
        engine.get_graph().set_grouping(grouping);
        const int n = 192;
        std::vector<sb::Tensor> bufs;
        unsigned x = seed;
        auto next = [&] { x = x * 1664525u + 1013904223u; return x >> 8; };
        for (int b = 0; b < nbuf; ++b)
        {
            bufs.push_back(engine.create_tensor({n, n}));
            std::vector<float> v(n * n);
            for (auto& e : v) e = float(int(next() % 2001) - 1000) / 1000.0f;
            fill_tensor(bufs.back(), v);
        }
        for (int i = 0; i < nops; ++i)
        {
            const int s1 = int(next() % nbuf), s2 = int(next() % nbuf);
            int d = int(next() % nbuf);
            while (d == s1 || d == s2) d = (d + 1) % nbuf;
            engine.blas().gemm(bufs[s1], bufs[s2], bufs[d], next() % 2 == 0, false, 0.01f, 0.5f);
        }
        engine.execute().wait();
        std::vector<float> out;
        for (auto& b : bufs) out.insert(out.end(), b.data_as<float>(), b.data_as<float>() + n * n);
        return out;
    }
} // namespace

TEST_CASE(RandomDagSameBitsOnOneOrFourLanes, true)
{
    // the in-order single lane is the reference schedule: every hazard the
    // multi-lane schedule misses shows up as different bits
    for (unsigned seed : {1u, 7u, 2026u})
    {
        const auto one = random_dag(1, 6, 60, seed);
        const auto four = random_dag(4, 6, 60, seed);
        CHECK(one.size() == four.size());
        CHECK(std::memcmp(one.data(), four.data(), one.size() * sizeof(float)) == 0);
    }
}

TEST_CASE(GroupedLaunchesMatchSingleLaunches, true)
{
    // grouping changes only how launches are formed (one batched launch may
    // pick another tile or split than a single one): same values to rounding
    for (unsigned seed : {3u, 11u})
    {
        const auto grouped = random_dag(4, 8, 80, seed, true);
        const auto single = random_dag(1, 8, 80, seed, false);
        double num = 0, den = 0;
        for (size_t i = 0; i < single.size(); ++i)
        {
            num += double(grouped[i] - single[i]) * (grouped[i] - single[i]);
            den += double(single[i]) * single[i];
        }
        CHECK(std::sqrt(num / den) <= 1e-5);
    }
}

TEST_CASE(GroupedRunsTraceEveryTaskAndStopAtHazards, true)
{
    sb::Engine engine(ctx());
    std::vector<std::string> names;
    engine.get_graph().set_trace_hook([&](const sr::Graph::TaskMetadata& m) { names.push_back(m.name); });
    const int N = 16, ops = 40;
    std::vector<sb::Tensor> A, C;
    auto B = engine.create_tensor({N, N});
    fill_tensor(B, std::vector<float>(N * N, 1.0f));
    for (int i = 0; i < ops; ++i)
    {
        A.push_back(engine.create_tensor({N, N}));
        C.push_back(engine.create_tensor({N, N}));
        fill_tensor(A.back(), std::vector<float>(N * N, float(i + 1)));
    }
    // 40 independent GEMMs (one grouped launch), then a GEMM that reads C[0]
    // (RAW on the run: must come after it), then 40 more reading C[i] into A[i]
    for (int i = 0; i < ops; ++i) engine.blas().gemm(A[i], B, C[i]);
    auto D = engine.create_tensor({N, N});
    engine.blas().gemm(C[0], B, D);
    for (int i = 0; i < ops; ++i) engine.blas().gemm(C[i], B, A[i], false, false, 0.5f, 0.0f);
    engine.execute().wait();
    CHECK(names.size() == size_t(2 * ops + 1));
    for (const auto& nm : names) CHECK(nm == "blas.lvl3.gemm");
    for (int i = 0; i < ops; ++i)
    {
        verify_tensor(C[i], std::vector<float>(N * N, float(N * (i + 1))), 0.0);
        verify_tensor(A[i], std::vector<float>(N * N, 0.5f * N * N * (i + 1)), 0.0);
    }
    verify_tensor(D, std::vector<float>(N * N, float(N * N)), 0.0);
}

TEST_CASE(CrossLaneRawAndWar, true)
{
    sb::Engine engine(ctx());
    std::vector<std::string> names;
    const int n = 1024;
    auto X = engine.create_tensor({n, n});
    auto W = engine.create_tensor({n, n});
    auto C0 = engine.create_tensor({n, n});
    auto U = engine.create_tensor({64, 64});
    auto V = engine.create_tensor({64, 64});
    auto D = engine.create_tensor({64, 64});
    std::vector<float> x(n * n), w(n * n);
    for (int i = 0; i < n * n; ++i)
    {
        x[i] = float((i * 7) % 13) - 6.0f;
        w[i] = float((i * 5) % 11) - 5.0f;
    }
    fill_tensor(X, x);
    fill_tensor(W, w);
    fill_tensor(U, std::vector<float>(64 * 64, 1.0f));
    fill_tensor(V, std::vector<float>(64 * 64, 2.0f));
    // T0 reads X (slow, 1024^3); T1 is independent (another lane); T2 reads
    // T1's D and overwrites X's first 64x64 block: it must wait for T0 on the
    // other lane (WAR) and for T1 (RAW)
    engine.blas().gemm(X, W, C0);
    engine.blas().gemm(U, V, D);
    sb::Tensor X64(X.storage, {64, 64});  // first 64*64 elements of X's storage
    engine.blas().gemm(D, V, X64);
    engine.execute().wait();
    // C0 from the original X, exact (small integers)
    const float* c0 = C0.data_as<float>();
    for (int i = 0; i < n; i += 97)
        for (int j = 0; j < n; j += 89)
        {
            double sacc = 0;
            for (int k = 0; k < n; ++k) sacc += double(x[i * n + k]) * w[k * n + j];
            CHECK(c0[i * n + j] == float(sacc));
        }
    // D = 1*2*64 = 128 everywhere, X64 = D*V = 128*2*64
    verify_tensor(D, std::vector<float>(64 * 64, 128.0f), 0.0);
    const float* xb = X.data_as<float>();
    for (int i = 0; i < 64 * 64; ++i) CHECK(xb[i] == 16384.0f);
}

TEST_CASE(LargeFp32MatchesHostLoop, true)
{
    // 300 x 257 x 129 with odd leading dimensions, against a double host loop
    sb::Engine engine(ctx());
    const int m = 300, n = 257, k = 129;
    auto A = engine.create_tensor({m, k});
    auto B = engine.create_tensor({k, n});
    auto C = engine.create_tensor({m, n});
    std::vector<float> a(m * k), b(k * n), c(m * n);
    for (int i = 0; i < m * k; ++i) a[i] = std::sin(0.37f * i);
    for (int i = 0; i < k * n; ++i) b[i] = std::cos(0.11f * i);
    for (int i = 0; i < m * n; ++i) c[i] = 0.25f * ((i % 9) - 4);
    fill_tensor(A, a);
    fill_tensor(B, b);
    fill_tensor(C, c);
    engine.blas().gemm(A, B, C, false, false, 1.25f, 0.5f);
    engine.execute().wait();
    double num = 0, den = 0;
    const float* got = C.data_as<float>();
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
        {
            double s = 0;
            for (int p = 0; p < k; ++p) s += double(a[i * k + p]) * b[p * n + j];
            const double want = 1.25 * s + 0.5 * c[i * n + j];
            num += (got[i * n + j] - want) * (got[i * n + j] - want);
            den += want * want;
        }
    CHECK(std::sqrt(num / den) <= 1e-5);
}

int main(int argc, char** argv)
{
    bool want_cpu = false, want_gpu = false, list = false;
    std::vector<std::string> names;
    for (int i = 1; i < argc; ++i)
    {
        std::string a = argv[i];
        if (a == "--cpu") want_cpu = true;
        else if (a == "--gpu") want_gpu = true;
        else if (a == "--list") list = true;
        else names.push_back(a);
    }
    if (!want_cpu && !want_gpu && names.empty()) want_cpu = want_gpu = true;
    int failed = 0, ran = 0;
    for (const Case& c : registry())
    {
        bool sel = (c.gpu ? want_gpu : want_cpu);
        for (const auto& n : names) sel = sel || n == c.name;
        if (!sel) continue;
        if (list)
        {
            std::printf("%s %s\n", c.gpu ? "gpu" : "cpu", c.name);
            continue;
        }
        ++ran;
        std::printf("[ RUN  ] %s\n", c.name);
        std::fflush(stdout);
        try
        {
            c.fn();
            std::printf("[  OK  ] %s\n", c.name);
        }
        catch (const Skip& k)
        {
            std::printf("[ SKIP ] %s: %s\n", c.name, k.why.c_str());
        }
        catch (const Failure& f)
        {
            ++failed;
            std::printf("[FAILED] %s: %s\n", c.name, f.what.c_str());
        }
        catch (const std::exception& e)
        {
            ++failed;
            std::printf("[FAILED] %s: exception: %s\n", c.name, e.what());
        }
        std::fflush(stdout);
    }
    if (!list) std::printf("%d cases, %d failed\n", ran, failed);
    return failed;
}
