// SushiRuntime.h -- the runtime surface SushiBLAS's GEMM path needs, on HIP.
//
// The reference's SushiRuntime ships as closed Windows binaries with public
// headers (include/SushiRuntime/**); this is a from-scratch stand-in for the
// part of that surface Level3::gemm and the Engine touch, with the same names
// so that SushiBLAS code and tests compile unchanged apart from the
// sycl::queue / sycl::event types:
//   Core::RefCounted, sushi_ptr, make_sushi   (core/ref_counted.hpp, core/sushi_ptr.hpp)
//   Memory::AllocStrategy, USMAllocator       (memory/usm_allocator.hpp:33-74)
//   Execution::RuntimeContext                 (execution/runtime_context.hpp:42-96)
//   Graph::OpID, TaskMetadata, TaskGraph      (graph/task_types.hpp, graph/task_graph.hpp)
// sycl::queue becomes Execution::Queue (one HIP stream, default priority) and
// sycl::event becomes Execution::Event (a HIP event; a default-constructed
// Event is already complete, like a default sycl::event).
//
// Scheduling: the reference's TaskGraph resolves read/write dependencies by
// base pointer and runs independent tasks in parallel on worker threads.  Here
// the same dependencies (RAW, WAW, WAR over the access sets' base pointers)
// place each task on one of a few HIP streams ("lanes") of the context:
// dependent tasks follow their latest dependency's lane or wait on an event
// recorded on the other lane, independent ones spread round-robin; execute()
// joins the lanes and returns an Event for the whole batch.
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <utility>
#include <vector>

namespace SushiRuntime
{
    namespace Core
    {
        /** @brief Allocation granularity of Storage (bytes). */
        inline constexpr size_t DEFAULT_ALIGNMENT = 128;
        inline constexpr size_t MAX_SUPPORTED_XPU = 16;

        /** @brief Intrusive reference count; the object deletes itself at zero. */
        class RefCounted
        {
            public:
                void add_ref() const noexcept { count_.fetch_add(1, std::memory_order_relaxed); }
                void release() const noexcept
                {
                    if (count_.fetch_sub(1, std::memory_order_acq_rel) == 1) delete this;
                }
                int ref_count() const noexcept { return count_.load(std::memory_order_acquire); }

            protected:
                RefCounted() = default;
                RefCounted(const RefCounted&) = delete;
                RefCounted& operator=(const RefCounted&) = delete;
                virtual ~RefCounted() = default;

            private:
                mutable std::atomic<int> count_{0};
        };
    } // namespace Core

    /** @brief Owning pointer to a Core::RefCounted object. */
    template <typename T>
    class sushi_ptr
    {
        public:
            sushi_ptr() noexcept = default;
            sushi_ptr(std::nullptr_t) noexcept {}
            sushi_ptr(T* p) : p_(p) { if (p_) p_->add_ref(); }
            sushi_ptr(const sushi_ptr& o) : sushi_ptr(o.p_) {}
            template <typename U, typename = std::enable_if_t<std::is_convertible_v<U*, T*>>>
            sushi_ptr(const sushi_ptr<U>& o) : sushi_ptr(static_cast<T*>(o.get())) {}
            sushi_ptr(sushi_ptr&& o) noexcept : p_(o.p_) { o.p_ = nullptr; }
            ~sushi_ptr() { if (p_) p_->release(); }

            sushi_ptr& operator=(sushi_ptr o) noexcept { std::swap(p_, o.p_); return *this; }
            void reset(T* p = nullptr) { sushi_ptr(p).swap(*this); }
            void swap(sushi_ptr& o) noexcept { std::swap(p_, o.p_); }

            T* get() const noexcept { return p_; }
            T* operator->() const noexcept { return p_; }
            T& operator*() const noexcept { return *p_; }
            explicit operator bool() const noexcept { return p_ != nullptr; }
            bool operator==(std::nullptr_t) const noexcept { return p_ == nullptr; }
            bool operator!=(std::nullptr_t) const noexcept { return p_ != nullptr; }
            bool operator==(const sushi_ptr& o) const noexcept { return p_ == o.p_; }
            bool operator!=(const sushi_ptr& o) const noexcept { return p_ != o.p_; }

        private:
            T* p_ = nullptr;
    };

    template <typename T, typename... Args>
    sushi_ptr<T> make_sushi(Args&&... args)
    {
        return sushi_ptr<T>(new T(std::forward<Args>(args)...));
    }

    namespace Execution
    {
        /** @brief Completion handle (stands in for sycl::event). */
        class Event
        {
            public:
                Event() = default;  // already complete
                explicit Event(hipStream_t stream);  // records on `stream`
                void wait() const;
                bool is_complete() const;
                hipEvent_t native() const { return ev_ ? ev_.get()->ev : nullptr; }

            private:
                struct Holder { hipEvent_t ev = nullptr; ~Holder(); };
                std::shared_ptr<Holder> ev_;
        };

        /** @brief One in-order HIP stream (stands in for sycl::queue). */
        class Queue
        {
            public:
                Queue(int device, hipStream_t stream) : device_(device), stream_(stream) {}
                hipStream_t native() const { return stream_; }
                int device() const { return device_; }
                void wait() const;
                Event record() const { return Event(stream_); }

            private:
                int device_;
                hipStream_t stream_;
        };
    } // namespace Execution

    namespace Memory
    {
        /** @brief Where an allocation lives (usm_allocator.hpp:33-38). */
        enum class AllocStrategy
        {
            DEVICE, /**< HBM only (hipMalloc); not host-addressable. */
            SHARED, /**< HBM + pinned host mirror, staged explicitly around execute(). */
            HOST    /**< Pinned host memory (hipHostMalloc), device-mapped. */
        };

        /** @brief Allocator interface (usm_allocator.hpp:43-71) plus the device
         *  address and staging hooks the HIP backend needs. */
        class USMAllocator : public Core::RefCounted
        {
            public:
                virtual void* allocate(size_t bytes, AllocStrategy strategy = AllocStrategy::SHARED,
                                       size_t alignment = Core::DEFAULT_ALIGNMENT) = 0;
                virtual void deallocate(void* ptr) = 0;
                /** @brief HIP device ordinal of an allocation (sycl::device in the reference). */
                virtual int get_device_of(void* ptr) = 0;
                /** @brief Address kernels use for an allocation's first byte. */
                virtual void* device_address(void* ptr) = 0;
                /** @brief Strategy of a live allocation (throws if unknown). */
                virtual AllocStrategy strategy_of(void* ptr) = 0;
                /** @brief True if `ptr` is the base of a live allocation. */
                virtual bool owns(void* ptr) = 0;
                /** @brief SHARED: copy host mirror -> device on `stream` (no-op otherwise). */
                virtual void upload(void* ptr, hipStream_t stream) = 0;
                /** @brief SHARED: copy device -> host mirror on `stream` (no-op otherwise). */
                virtual void download(void* ptr, hipStream_t stream) = 0;
        };

        /** @brief HIP allocator for one device. */
        sushi_ptr<USMAllocator> create_allocator(int device);
    } // namespace Memory

    namespace Execution
    {
        /** @brief Owns the HIP device, its streams and allocator
         *  (execution/runtime_context.hpp:42-96).  The device is touched on
         *  first use (std::call_once), so a context -- and an Engine over it --
         *  can be built, and GEMM arguments validated, on a host without a GPU. */
        class RuntimeContext
        {
            public:
                /** @brief Uses HIP device 0 (or $SBX_DEVICE). */
                RuntimeContext();
                explicit RuntimeContext(int device);
                ~RuntimeContext();
                RuntimeContext(const RuntimeContext&) = delete;
                RuntimeContext& operator=(const RuntimeContext&) = delete;

                Queue& get_queue(size_t xpu_index = 0);
                sushi_ptr<Memory::USMAllocator> get_allocator();
                int device() const { return device_; }
                /** @brief Wait for every lane of the device. */
                void wait_all();

                /** @brief Streams the task graph spreads independent tasks over
                 *  (stands in for the reference's worker threads,
                 *  task_scheduler.hpp:79).  Lane 0 is get_queue(0). */
                static constexpr size_t kLanes = 4;
                Queue& get_lane(size_t lane);

            private:
                void init();
                int device_ = 0;
                std::once_flag once_;
                hipStream_t streams_[kLanes] = {};
                std::unique_ptr<Queue> lanes_[kLanes];
                sushi_ptr<Memory::USMAllocator> allocator_;
        };
    } // namespace Execution

    namespace Graph
    {
        /** @brief Operation identifier: 32-bit FNV-1a of the op name
         *  (graph/task_types.hpp:58-83), so ids match the reference's. */
        struct OpID
        {
            uint32_t value = 0;
            constexpr OpID() = default;
            constexpr explicit OpID(uint32_t v) : value(v) {}
            static constexpr uint32_t hash_str(const char* s, size_t n)
            {
                uint32_t h = 2166136261u;
                for (size_t i = 0; i < n; ++i)
                {
                    h ^= static_cast<uint32_t>(static_cast<unsigned char>(s[i]));
                    h *= 16777619u;
                }
                return h;
            }
            constexpr bool operator==(const OpID& o) const { return value == o.value; }
            constexpr bool operator!=(const OpID& o) const { return value != o.value; }
        };

        namespace Literals
        {
            constexpr OpID operator""_op(const char* s, size_t n) { return OpID(OpID::hash_str(s, n)); }
        }

        enum class TaskType { NONE, MATH_OP, MEMORY_OP, CUSTOM_HOST, CONTROL_FLOW };

        /** @brief Profiler-facing description of a task (graph/task_types.hpp:90-129). */
        struct TaskMetadata
        {
            const char* name = "unnamed_task";
            TaskType task_type = TaskType::NONE;
            OpID op_id = OpID(0);
            static constexpr size_t K_MAX_PARAMS = 8;
            uint64_t params[K_MAX_PARAMS] = {0};

            template <typename T>
            void set_param(int index, T value)
            {
                static_assert(std::is_trivially_copyable_v<T> && sizeof(T) <= sizeof(uint64_t),
                              "parameter must be a trivially copyable value of at most 64 bits");
                if (index >= 0 && index < static_cast<int>(K_MAX_PARAMS))
                {
                    params[index] = 0;
                    std::memcpy(&params[index], &value, sizeof(T));
                }
            }

            template <typename T>
            T get_param(int index) const
            {
                static_assert(std::is_trivially_copyable_v<T> && sizeof(T) <= sizeof(uint64_t),
                              "parameter must be a trivially copyable value of at most 64 bits");
                T value{};
                if (index >= 0 && index < static_cast<int>(K_MAX_PARAMS))
                    std::memcpy(&value, &params[index], sizeof(T));
                return value;
            }
        };

        /** @brief Deferred task body (HostWork, graph/task_graph.hpp:46). */
        using HostWork = std::function<Execution::Event(Execution::Queue&,
                                                        const std::vector<Execution::Event>&)>;

        /** @brief Optional observer called for each task as it is issued. */
        using TraceHook = std::function<void(const TaskMetadata&)>;

        /** @brief What a fuser needs to know about a task (the reference's
         *  TaskMetadata is meant "for profilers/fusers", gemm.cpp:126; this
         *  backend implements one fusion: a GEMM immediately followed by a ReLU
         *  on exactly its output runs as one kernel with a ReLU epilogue). */
        struct FusionHook
        {
            enum Kind { NONE, PRODUCER, RELU } kind = NONE;
            void* base = nullptr;     // storage base pointer of the output region
            size_t offset_bytes = 0;  // first byte of the region in that storage
            int64_t elements = 0;     // contiguous elements in the region
            int dtype = -1;           // element type tag
            HostWork with_relu;       // PRODUCER: the same work with the ReLU fused
            const char* fused_name = nullptr;  // PRODUCER: task name once fused
        };

        /** @brief Grouping description of a task: consecutive independent
         *  tasks with equal `key`s (same launch parameters) are issued as one
         *  launch over a device table of their operand pointers. */
        struct GroupHook
        {
            bool enabled = false;
            uint64_t key[8] = {};
            const void* ptrs[3] = {};  // this task's A, B, C device addresses
            bool aligned = false;      // all three 16-byte aligned
            int epilogue = 0;          // 1 once a ReLU has been fused into the task
            /** Issue `count` problems whose pointers are at `table` (device). */
            std::function<void(Execution::Queue&, const void* const* table, int64_t count,
                               bool aligned, int epilogue)>
                launch;
        };

        /** @brief A task as the grouping planner sees it. */
        struct GroupCandidate
        {
            const GroupHook* group = nullptr;  // null or !enabled: not groupable
            bool has_deps = false;             // explicit event dependencies
            const std::vector<void*>* reads = nullptr;
            const std::vector<void*>* writes = nullptr;
        };

        /** @brief One run of tasks issued as a single grouped launch. */
        struct GroupRun
        {
            size_t first = 0;        // index of the first task
            size_t count = 0;        // tasks (>= 2)
            int64_t table_offset = 0;  // first problem in the table (3 pointers each)
            bool aligned = true;     // every pointer 16-byte aligned
        };

        /** @brief Runs of consecutive groupable tasks with equal keys and
         *  epilogues and no hazard among them, and the pointer table (A, B, C
         *  per task, in task order) that their launches read. */
        std::vector<GroupRun> plan_groups(const std::vector<GroupCandidate>& tasks,
                                          std::vector<const void*>& table);

        /** @brief Record-then-execute task list (graph/task_graph.hpp:55-124). */
        class TaskGraph
        {
            public:
                explicit TaskGraph(Execution::RuntimeContext& ctx) : ctx_(ctx) {}
                ~TaskGraph();
                TaskGraph(const TaskGraph&) = delete;
                TaskGraph& operator=(const TaskGraph&) = delete;

                /** @brief Record a task.  `read_access` / `write_access` are base
                 *  pointers of Storage allocations (gemm.cpp:112-120); SHARED ones
                 *  are staged to the device before the batch and written ones
                 *  back to the host mirror after it. */
                void add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                              const std::vector<void*>& write_access, HostWork work,
                              const std::vector<Execution::Event>& dependencies = {});

                /** @brief As above, with the task's fusion description. */
                void add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                              const std::vector<void*>& write_access, HostWork work,
                              FusionHook fusion,
                              const std::vector<Execution::Event>& dependencies = {});

                /** @brief As above, with fusion and grouping descriptions. */
                void add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                              const std::vector<void*>& write_access, HostWork work,
                              FusionHook fusion, GroupHook group,
                              const std::vector<Execution::Event>& dependencies = {});

                /** @brief Issue every recorded task; returns an Event that completes
                 *  when all of them (and the staging copies) have.
                 *  Dependencies come from the access sets, as in the reference
                 *  (task_graph.hpp:107-117): a task waits for the last writer of
                 *  everything it reads or writes and for every reader of what it
                 *  writes since that write (RAW, WAW, WAR).  Independent tasks are
                 *  spread over the context's lanes (HIP streams); a task runs on
                 *  the lane of its latest dependency, so chains stay in one
                 *  stream, and a dependency on another lane becomes an event
                 *  wait.  Trace hooks see the tasks in record order.  A
                 *  PRODUCER task directly followed by a RELU task over the same
                 *  region (same base, offset, element count and type, no extra
                 *  dependencies) is issued once, as its fused form. */
                Execution::Event execute();

                size_t pending() const;
                void set_trace_hook(TraceHook hook);
                /** @brief Turn GEMM+ReLU fusion on (default) or off. */
                void set_fusion(bool enabled);
                /** @brief Use at most `lanes` streams (1 = strictly in order). */
                void set_max_lanes(size_t lanes);
                /** @brief Turn grouped launches of same-shaped independent tasks
                 *  on (default) or off. */
                void set_grouping(bool enabled);

            private:
                struct Task
                {
                    TaskMetadata meta;
                    std::vector<void*> reads, writes;
                    HostWork work;
                    std::vector<Execution::Event> deps;
                    FusionHook fusion;
                    GroupHook group;
                    // a grouped task: the members' metadata (for the trace hook)
                    // and its slice of the batch's pointer table
                    std::vector<TaskMetadata> members;
                    int64_t table_offset = -1;  // first problem (3 pointers each)
                    int64_t table_count = 0;    // problems
                    bool table_aligned = false;
                };
                Execution::RuntimeContext& ctx_;
                mutable std::mutex mu_;
                std::vector<Task> tasks_;
                TraceHook trace_;
                bool fusion_ = true;
                size_t max_lanes_ = Execution::RuntimeContext::kLanes;
                size_t next_lane_ = 0;
                hipEvent_t lane_events_[Execution::RuntimeContext::kLanes] = {};
                bool grouping_ = true;
                // pointer tables of grouped tasks: pinned staging -> device,
                // one copy per batch on lane 0
                void* table_dev_ = nullptr;
                void* table_pin_ = nullptr;
                size_t table_cap_ = 0;  // pointers
                hipEvent_t table_copied_ = nullptr;
        };
    } // namespace Graph
} // namespace SushiRuntime

namespace sr = SushiRuntime;
