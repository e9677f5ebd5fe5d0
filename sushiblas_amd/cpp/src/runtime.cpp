// runtime.cpp -- HIP implementation of the SushiRuntime surface used by the
// GEMM path: events, the streams, the allocator with explicit host<->device
// staging for SHARED allocations, the context and the task graph.
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
                // default priority on every lane: streams of mixed priorities
                // are avoided on purpose
                for (size_t i = 0; i < kLanes; ++i)
                {
                    check(hipStreamCreateWithFlags(&streams_[i], hipStreamNonBlocking),
                          "hipStreamCreate");
                    lanes_[i] = std::make_unique<Queue>(device_, streams_[i]);
                }
                allocator_ = Memory::create_allocator(device_);
            });
        }

        RuntimeContext::~RuntimeContext()
        {
            for (size_t i = 0; i < kLanes; ++i)
                if (streams_[i])
                {
                    (void)hipStreamSynchronize(streams_[i]);
                    (void)hipStreamDestroy(streams_[i]);
                }
        }

        Queue& RuntimeContext::get_lane(size_t lane)
        {
            if (lane >= kLanes) throw std::runtime_error("RuntimeContext: no such lane");
            init();
            return *lanes_[lane];
        }

        Queue& RuntimeContext::get_queue(size_t xpu_index)
        {
            if (xpu_index != 0)
                throw std::runtime_error("RuntimeContext: this build drives one device (xpu 0)");
            init();
            return *lanes_[0];
        }

        sushi_ptr<Memory::USMAllocator> RuntimeContext::get_allocator()
        {
            init();
            return allocator_;
        }

        void RuntimeContext::wait_all()
        {
            for (size_t i = 0; i < kLanes; ++i)
                if (lanes_[i]) lanes_[i]->wait();
        }
    } // namespace Execution

    // ----------------------------------------------------------- task graph
    namespace Graph
    {
        void TaskGraph::add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                                 const std::vector<void*>& write_access, HostWork work,
                                 const std::vector<Execution::Event>& dependencies)
        {
            add_task(meta, read_access, write_access, std::move(work), FusionHook{}, GroupHook{},
                     dependencies);
        }

        void TaskGraph::add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                                 const std::vector<void*>& write_access, HostWork work,
                                 FusionHook fusion,
                                 const std::vector<Execution::Event>& dependencies)
        {
            add_task(meta, read_access, write_access, std::move(work), std::move(fusion),
                     GroupHook{}, dependencies);
        }

        void TaskGraph::add_task(const TaskMetadata& meta, const std::vector<void*>& read_access,
                                 const std::vector<void*>& write_access, HostWork work,
                                 FusionHook fusion, GroupHook group,
                                 const std::vector<Execution::Event>& dependencies)
        {
            Task t;
            t.meta = meta;
            t.reads = read_access;
            t.writes = write_access;
            t.work = std::move(work);
            t.deps = dependencies;
            t.fusion = std::move(fusion);
            t.group = std::move(group);
            std::lock_guard<std::mutex> g(mu_);
            tasks_.push_back(std::move(t));
        }

        void TaskGraph::set_grouping(bool enabled)
        {
            std::lock_guard<std::mutex> g(mu_);
            grouping_ = enabled;
        }

        void TaskGraph::set_fusion(bool enabled)
        {
            std::lock_guard<std::mutex> g(mu_);
            fusion_ = enabled;
        }

        void TaskGraph::set_max_lanes(size_t lanes)
        {
            std::lock_guard<std::mutex> g(mu_);
            max_lanes_ = lanes < 1 ? 1 : (lanes > Execution::RuntimeContext::kLanes
                                              ? Execution::RuntimeContext::kLanes
                                              : lanes);
        }

        TaskGraph::~TaskGraph()
        {
            for (hipEvent_t e : lane_events_)
                if (e) (void)hipEventDestroy(e);
            if (table_dev_ || table_pin_)
            {
                ctx_.wait_all();  // grouped kernels may still read the table
                if (table_dev_) (void)hipFree(table_dev_);
                if (table_pin_) (void)hipHostFree(table_pin_);
            }
            if (table_copied_) (void)hipEventDestroy(table_copied_);
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

        std::vector<GroupRun> plan_groups(const std::vector<GroupCandidate>& tasks,
                                          std::vector<const void*>& table)
        {
            std::vector<GroupRun> runs;
            table.clear();
            auto groupable = [&](size_t i) {
                const GroupCandidate& c = tasks[i];
                return c.group && c.group->enabled && !c.has_deps && c.group->launch;
            };
            for (size_t i = 0; i < tasks.size();)
            {
                size_t j = i + 1;
                if (groupable(i))
                {
                    const GroupHook& head = *tasks[i].group;
                    std::unordered_set<void*> run_w(tasks[i].writes->begin(), tasks[i].writes->end());
                    std::unordered_set<void*> run_rw(run_w);
                    run_rw.insert(tasks[i].reads->begin(), tasks[i].reads->end());
                    while (j < tasks.size() && groupable(j))
                    {
                        const GroupHook& g = *tasks[j].group;
                        if (g.epilogue != head.epilogue ||
                            std::memcmp(g.key, head.key, sizeof(head.key)) != 0)
                            break;
                        bool hazard = false;
                        for (void* p : *tasks[j].writes) hazard = hazard || run_rw.count(p);
                        for (void* p : *tasks[j].reads) hazard = hazard || run_w.count(p);
                        if (hazard) break;
                        run_w.insert(tasks[j].writes->begin(), tasks[j].writes->end());
                        run_rw.insert(tasks[j].writes->begin(), tasks[j].writes->end());
                        run_rw.insert(tasks[j].reads->begin(), tasks[j].reads->end());
                        ++j;
                    }
                }
                if (j - i >= 2)
                {
                    GroupRun r;
                    r.first = i;
                    r.count = j - i;
                    r.table_offset = static_cast<int64_t>(table.size() / 3);
                    for (size_t q = i; q < j; ++q)
                    {
                        const GroupHook& g = *tasks[q].group;
                        for (int e = 0; e < 3; ++e) table.push_back(g.ptrs[e]);
                        r.aligned = r.aligned && g.aligned;
                    }
                    runs.push_back(r);
                }
                i = j;
            }
            return runs;
        }

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
                    t.group.epilogue = 1;
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
            Execution::Queue& main = ctx_.get_queue();
            if (tasks.empty()) return main.record();
            auto alloc = ctx_.get_allocator();
            check(hipSetDevice(main.device()), "hipSetDevice");
            size_t lanes;
            bool group_on;
            {
                std::lock_guard<std::mutex> g(mu_);
                lanes = max_lanes_;
                group_on = grouping_;
            }

            // Runs of consecutive grouped-launch candidates with equal keys and no
            // hazard among them become one task over a slice of a pointer table.
            std::vector<const void*> table;
            if (group_on)
            {
                std::vector<GroupCandidate> cand(tasks.size());
                for (size_t i = 0; i < tasks.size(); ++i)
                    cand[i] = GroupCandidate{&tasks[i].group, !tasks[i].deps.empty(), &tasks[i].reads,
                                             &tasks[i].writes};
                const std::vector<GroupRun> runs = plan_groups(cand, table);
                std::vector<Task> merged;
                merged.reserve(tasks.size());
                size_t next = 0;
                for (const GroupRun& r : runs)
                {
                    for (; next < r.first; ++next) merged.push_back(std::move(tasks[next]));
                    Task g;
                    g.meta = tasks[r.first].meta;
                    g.group = tasks[r.first].group;
                    g.table_offset = r.table_offset;
                    g.table_count = static_cast<int64_t>(r.count);
                    g.table_aligned = r.aligned;
                    std::unordered_set<void*> rs, ws;
                    for (size_t q = r.first; q < r.first + r.count; ++q)
                    {
                        Task& t = tasks[q];
                        g.members.push_back(t.meta);
                        for (void* p : t.reads)
                            if (rs.insert(p).second) g.reads.push_back(p);
                        for (void* p : t.writes)
                            if (ws.insert(p).second) g.writes.push_back(p);
                    }
                    merged.push_back(std::move(g));
                    next = r.first + r.count;
                }
                for (; next < tasks.size(); ++next) merged.push_back(std::move(tasks[next]));
                tasks.swap(merged);
            }
            const void* const* table_dev = nullptr;
            if (!table.empty())
            {
                // the previous batch's copy must be done before the staging
                // buffer is rewritten; lane 0 orders the device copy after the
                // previous batch's kernels (they were joined into lane 0)
                if (table_copied_) check(hipEventSynchronize(table_copied_), "hipEventSynchronize");
                if (table.size() > table_cap_)
                {
                    ctx_.wait_all();
                    if (table_dev_) (void)hipFree(table_dev_);
                    if (table_pin_) (void)hipHostFree(table_pin_);
                    table_dev_ = table_pin_ = nullptr;
                    table_cap_ = 0;
                    const size_t cap = table.size() * 2;
                    check(hipMalloc(&table_dev_, cap * sizeof(void*)), "hipMalloc");
                    check(hipHostMalloc(&table_pin_, cap * sizeof(void*), hipHostMallocDefault),
                          "hipHostMalloc");
                    table_cap_ = cap;
                }
                if (!table_copied_)
                    check(hipEventCreateWithFlags(&table_copied_, hipEventDisableTiming),
                          "hipEventCreate");
                std::memcpy(table_pin_, table.data(), table.size() * sizeof(void*));
                check(hipMemcpyAsync(table_dev_, table_pin_, table.size() * sizeof(void*),
                                     hipMemcpyHostToDevice, main.native()),
                      "hipMemcpyAsync(table)");
                check(hipEventRecord(table_copied_, main.native()), "hipEventRecord");
                table_dev = static_cast<const void* const*>(table_dev_);
            }
            for (size_t i = 0; i < lanes; ++i)
                if (!lane_events_[i])
                    check(hipEventCreateWithFlags(&lane_events_[i], hipEventDisableTiming),
                          "hipEventCreate");
            // Make lane `to` wait for everything issued so far on lane `from`.
            auto join = [&](size_t to, size_t from) {
                if (to == from) return;
                hipStream_t src = ctx_.get_lane(from).native();
                check(hipEventRecord(lane_events_[from], src), "hipEventRecord");
                check(hipStreamWaitEvent(ctx_.get_lane(to).native(), lane_events_[from], 0),
                      "hipStreamWaitEvent");
            };

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
            for (void* p : staged) alloc->upload(p, main.native());
            // a lane other than 0 waits for the uploads (and the pointer table)
            // when it is first used, and lane 0 waits for every other lane that
            // was used at the end
            const bool copies_on_main = !staged.empty() || !table.empty();
            bool used[Execution::RuntimeContext::kLanes] = {};
            used[0] = true;
            auto use = [&](size_t lane) {
                if (used[lane]) return;
                used[lane] = true;
                if (copies_on_main) join(lane, 0);
            };

            // Hazards by base pointer: the last writer, and the readers since it.
            struct Access
            {
                long writer = -1;
                std::vector<long> readers;
            };
            std::unordered_map<void*, Access> acc;
            std::vector<size_t> lane_of(tasks.size(), 0);
            next_lane_ = 0;  // a batch that is one chain stays on lane 0: no joins
            for (size_t i = 0; i < tasks.size(); ++i)
            {
                Task& t = tasks[i];
                std::vector<long> deps;
                for (void* p : t.reads)
                    if (p)
                    {
                        auto it = acc.find(p);
                        if (it != acc.end() && it->second.writer >= 0) deps.push_back(it->second.writer);
                    }
                for (void* p : t.writes)
                    if (p)
                    {
                        auto it = acc.find(p);
                        if (it == acc.end()) continue;
                        if (it->second.writer >= 0) deps.push_back(it->second.writer);
                        deps.insert(deps.end(), it->second.readers.begin(), it->second.readers.end());
                    }
                // the lane of the latest dependency, else the next lane in turn
                size_t lane;
                if (!deps.empty())
                {
                    long latest = deps[0];
                    for (long d : deps) latest = d > latest ? d : latest;
                    lane = lane_of[latest];
                }
                else
                {
                    lane = next_lane_ % lanes;
                    next_lane_ = (next_lane_ + 1) % lanes;
                }
                // one wait per other lane that holds a dependency
                bool waited[Execution::RuntimeContext::kLanes] = {};
                for (long d : deps)
                    if (lane_of[d] != lane && !waited[lane_of[d]])
                    {
                        join(lane, lane_of[d]);
                        waited[lane_of[d]] = true;
                    }
                use(lane);
                lane_of[i] = lane;
                Execution::Queue& q = ctx_.get_lane(lane);
                for (const Execution::Event& d : t.deps)
                    if (d.native()) check(hipStreamWaitEvent(q.native(), d.native(), 0), "hipStreamWaitEvent");
                if (t.table_offset >= 0)
                {
                    // the slice must lie inside the table copied for this batch
                    if (!table_dev || t.table_count < 1 ||
                        static_cast<size_t>(3 * (t.table_offset + t.table_count)) > table.size())
                        throw std::runtime_error("TaskGraph: grouped task outside its pointer table");
                    if (trace)
                        for (const TaskMetadata& m : t.members) trace(m);
                    t.group.launch(q, table_dev + 3 * t.table_offset, t.table_count,
                                   t.table_aligned, t.group.epilogue);
                }
                else
                {
                    if (trace) trace(t.meta);
                    t.work(q, t.deps);
                }
                // record the accesses
                for (void* p : t.reads)
                    if (p) acc[p].readers.push_back(static_cast<long>(i));
                for (void* p : t.writes)
                    if (p)
                    {
                        Access& a = acc[p];
                        a.writer = static_cast<long>(i);
                        a.readers.clear();
                    }
            }
            for (size_t l = 1; l < lanes; ++l)
                if (used[l]) join(0, l);
            for (void* p : written) alloc->download(p, main.native());
            return main.record();
        }
    } // namespace Graph
} // namespace SushiRuntime
