// runtime.cpp -- HIP implementation of the SushiRuntime surface used by the
// GEMM path: events, the stream, the allocator with explicit host<->device
// staging for SHARED allocations, the context and the in-order task list.
#include <SushiRuntime/SushiRuntime.h>

#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_set>

namespace SushiRuntime
{
    namespace
    {
        void check(hipError_t e, const char* what)
        {
            if (e != hipSuccess)
                throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
        }
    } // namespace

    // ---------------------------------------------------------------- Event
    namespace Execution
    {
        Event::Holder::~Holder()
        {
            if (ev) (void)hipEventDestroy(ev);
        }

        Event::Event(hipStream_t stream) : ev_(std::make_shared<Holder>())
        {
            check(hipEventCreateWithFlags(&ev_->ev, hipEventDisableTiming), "hipEventCreate");
            check(hipEventRecord(ev_->ev, stream), "hipEventRecord");
        }

        void Event::wait() const
        {
            if (ev_) check(hipEventSynchronize(ev_->ev), "hipEventSynchronize");
        }

        bool Event::is_complete() const
        {
            if (!ev_) return true;
            hipError_t e = hipEventQuery(ev_->ev);
            if (e == hipErrorNotReady) return false;
            check(e, "hipEventQuery");
            return true;
        }

        void Queue::wait() const { check(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }
    } // namespace Execution

    // ------------------------------------------------------------ allocator
    namespace Memory
    {
        namespace
        {
            struct Block
            {
                AllocStrategy strategy;
                void* host = nullptr;    // SHARED mirror / HOST memory
                void* device = nullptr;  // what kernels use
                size_t bytes = 0;
            };

            /** @brief hipMalloc / hipHostMalloc backed allocator for one device.
             *  SHARED = HBM buffer + pinned host mirror: the pointer handed out
             *  is the mirror (host code writes through it, as the reference's
             *  tests do with USM shared memory), and TaskGraph::execute stages
             *  it explicitly. */
            class HipAllocator final : public USMAllocator
            {
                public:
                    explicit HipAllocator(int device) : device_(device) {}

                    void* allocate(size_t bytes, AllocStrategy strategy, size_t alignment) override
                    {
                        if (bytes == 0) return nullptr;
                        if (alignment > 256 || (alignment & (alignment - 1)))
                            throw std::runtime_error("USMAllocator: unsupported alignment");
                        check(hipSetDevice(device_), "hipSetDevice");
                        Block b;
                        b.strategy = strategy;
                        b.bytes = bytes;
                        void* handle = nullptr;
                        switch (strategy)
                        {
                            case AllocStrategy::DEVICE:
                                check(hipMalloc(&b.device, bytes), "hipMalloc");
                                handle = b.device;
                                break;
                            case AllocStrategy::HOST:
                                check(hipHostMalloc(&b.host, bytes, hipHostMallocDefault),
                                      "hipHostMalloc");
                                check(hipHostGetDevicePointer(&b.device, b.host, 0),
                                      "hipHostGetDevicePointer");
                                handle = b.host;
                                break;
                            case AllocStrategy::SHARED:
                                check(hipMalloc(&b.device, bytes), "hipMalloc");
                                if (hipHostMalloc(&b.host, bytes, hipHostMallocDefault) != hipSuccess)
                                {
                                    (void)hipFree(b.device);
                                    throw std::runtime_error("hipHostMalloc failed for a SHARED mirror");
                                }
                                handle = b.host;
                                break;
                        }
                        std::lock_guard<std::mutex> g(mu_);
                        blocks_[handle] = b;
                        return handle;
                    }

                    void deallocate(void* ptr) override
                    {
                        Block b;
                        {
                            std::lock_guard<std::mutex> g(mu_);
                            auto it = blocks_.find(ptr);
                            if (it == blocks_.end()) return;
                            b = it->second;
                            blocks_.erase(it);
                        }
                        (void)hipSetDevice(device_);
                        if (b.strategy == AllocStrategy::HOST)
                        {
                            (void)hipHostFree(b.host);
                            return;
                        }
                        // a kernel may still be reading the buffer: drain first
                        (void)hipDeviceSynchronize();
                        (void)hipFree(b.device);
                        if (b.host) (void)hipHostFree(b.host);
                    }

                    int get_device_of(void* ptr) override
                    {
                        find(ptr);
                        return device_;
                    }

                    void* device_address(void* ptr) override { return find(ptr).device; }
                    AllocStrategy strategy_of(void* ptr) override { return find(ptr).strategy; }

                    bool owns(void* ptr) override
                    {
                        std::lock_guard<std::mutex> g(mu_);
                        return blocks_.count(ptr) != 0;
                    }

                    void upload(void* ptr, hipStream_t stream) override
                    {
                        Block b = find(ptr);
                        if (b.strategy != AllocStrategy::SHARED) return;
                        check(hipMemcpyAsync(b.device, b.host, b.bytes, hipMemcpyHostToDevice, stream),
                              "hipMemcpyAsync(H2D)");
                    }

                    void download(void* ptr, hipStream_t stream) override
                    {
                        Block b = find(ptr);
                        if (b.strategy != AllocStrategy::SHARED) return;
                        check(hipMemcpyAsync(b.host, b.device, b.bytes, hipMemcpyDeviceToHost, stream),
                              "hipMemcpyAsync(D2H)");
                    }

                private:
                    Block find(void* ptr)
                    {
                        std::lock_guard<std::mutex> g(mu_);
                        auto it = blocks_.find(ptr);
                        if (it == blocks_.end())
                            throw std::runtime_error("USMAllocator: pointer is not a live allocation");
                        return it->second;
                    }

                    int device_;
                    std::mutex mu_;
                    std::unordered_map<void*, Block> blocks_;
            };
        } // namespace

        sushi_ptr<USMAllocator> create_allocator(int device)
        {
            return sushi_ptr<USMAllocator>(new HipAllocator(device));
        }
    } // namespace Memory

    // -------------------------------------------------------------- context
    namespace Execution
    {
        namespace
        {
            int default_device()
            {
                const char* env = std::getenv("SBX_DEVICE");
                return env ? std::atoi(env) : 0;
            }
        } // namespace

        RuntimeContext::RuntimeContext() : RuntimeContext(default_device()) {}

        RuntimeContext::RuntimeContext(int device) : device_(device) {}

        void RuntimeContext::init()
        {
            std::call_once(once_, [this] {
                check(hipSetDevice(device_), "hipSetDevice");
                check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
                queue_ = std::make_unique<Queue>(device_, stream_);
                allocator_ = Memory::create_allocator(device_);
            });
        }

        RuntimeContext::~RuntimeContext()
        {
            if (stream_)
            {
                (void)hipStreamSynchronize(stream_);
                (void)hipStreamDestroy(stream_);
            }
        }

        Queue& RuntimeContext::get_queue(size_t xpu_index)
        {
            if (xpu_index != 0)
                throw std::runtime_error("RuntimeContext: this build drives one device (xpu 0)");
            init();
            return *queue_;
        }

        sushi_ptr<Memory::USMAllocator> RuntimeContext::get_allocator()
        {
            init();
            return allocator_;
        }

        void RuntimeContext::wait_all()
        {
            if (queue_) queue_->wait();
        }
    } // namespace Execution

    // ----------------------------------------------------------- task graph
    namespace Graph
    {
        void TaskGraph::add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                                 const std::vector<void*>& write_access, HostWork work,
                                 const std::vector<Execution::Event>& dependencies)
        {
            add_task(meta, read_access, write_access, std::move(work), FusionHook{}, dependencies);
        }

        void TaskGraph::add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                                 const std::vector<void*>& write_access, HostWork work,
                                 FusionHook fusion,
                                 const std::vector<Execution::Event>& dependencies)
        {
            std::lock_guard<std::mutex> g(mu_);
            tasks_.push_back(Task{meta, read_access, write_access, std::move(work), dependencies,
                                  std::move(fusion)});
        }

        void TaskGraph::set_fusion(bool enabled)
        {
            std::lock_guard<std::mutex> g(mu_);
            fusion_ = enabled;
        }

        size_t TaskGraph::pending() const
        {
            std::lock_guard<std::mutex> g(mu_);
            return tasks_.size();
        }

        void TaskGraph::set_trace_hook(TraceHook hook)
        {
            std::lock_guard<std::mutex> g(mu_);
            trace_ = std::move(hook);
        }

        namespace
        {
            // A producer and the ReLU right after it cover the same elements:
            // running the producer's fused form instead of the pair writes the
            // same values and saves the ReLU's read and write of the region.
            bool fusable(const FusionHook& producer, const FusionHook& relu,
                         const std::vector<Execution::Event>& relu_deps)
            {
                return producer.kind == FusionHook::PRODUCER && relu.kind == FusionHook::RELU &&
                       producer.with_relu && producer.base && producer.base == relu.base &&
                       producer.offset_bytes == relu.offset_bytes &&
                       producer.elements == relu.elements && producer.elements > 0 &&
                       producer.dtype == relu.dtype && relu_deps.empty();
            }
        } // namespace

        Execution::Event TaskGraph::execute()
        {
            std::vector<Task> recorded, tasks;
            TraceHook trace;
            bool fuse = true;
            {
                std::lock_guard<std::mutex> g(mu_);
                recorded.swap(tasks_);
                trace = trace_;
                fuse = fusion_;
            }
            tasks.reserve(recorded.size());
            for (size_t i = 0; i < recorded.size(); ++i)
            {
                if (fuse && i + 1 < recorded.size() &&
                    fusable(recorded[i].fusion, recorded[i + 1].fusion, recorded[i + 1].deps))
                {
                    Task t = std::move(recorded[i]);
                    t.work = std::move(t.fusion.with_relu);
                    if (t.fusion.fused_name)
                    {
                        t.meta.name = t.fusion.fused_name;
                        t.meta.op_id = OpID(OpID::hash_str(t.fusion.fused_name,
                                                           std::strlen(t.fusion.fused_name)));
                    }
                    t.fusion = FusionHook{};
                    tasks.push_back(std::move(t));
                    ++i;
                    continue;
                }
                tasks.push_back(std::move(recorded[i]));
            }
            Execution::Queue& q = ctx_.get_queue();
            if (tasks.empty()) return q.record();
            auto alloc = ctx_.get_allocator();
            check(hipSetDevice(q.device()), "hipSetDevice");

            // SHARED allocations touched by the batch, in first-use order
            std::vector<void*> staged, written;
            std::unordered_set<void*> seen, seen_w;
            for (const Task& t : tasks)
            {
                for (const auto* list : {&t.reads, &t.writes})
                    for (void* p : *list)
                        if (p && !seen.count(p) && alloc->owns(p) &&
                            alloc->strategy_of(p) == Memory::AllocStrategy::SHARED)
                        {
                            seen.insert(p);
                            staged.push_back(p);
                        }
                for (void* p : t.writes)
                    if (p && seen.count(p) && !seen_w.count(p))
                    {
                        seen_w.insert(p);
                        written.push_back(p);
                    }
            }
            for (void* p : staged) alloc->upload(p, q.native());
            for (Task& t : tasks)
            {
                for (const Execution::Event& d : t.deps)
                    if (d.native()) check(hipStreamWaitEvent(q.native(), d.native(), 0), "hipStreamWaitEvent");
                if (trace) trace(t.meta);
                t.work(q, t.deps);
            }
            for (void* p : written) alloc->download(p, q.native());
            return q.record();
        }
    } // namespace Graph
} // namespace SushiRuntime
