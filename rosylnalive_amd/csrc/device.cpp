// The HIP device (see device.hpp). Follows the reference's contract for IGpuBackend / IGpuHeap / ICommandList
// (docs/contracts/gpu-backend.md, src/Lrm.Gpu.Core/Backend.fs:104-161) on one in-order HIP stream.
#include "device.hpp"

#include <dlfcn.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>

#include "sha256.hpp"

namespace lrm {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        char buf[512];
        snprintf(buf, sizeof buf, "%s: %s (%d)", what, hipGetErrorString(e), int(e));
        throw HipError(buf);
    }
}

#define HIPC(x) hip_check((x), #x)

// ---------------------------------------------------------------- enumeration

static uint32_t read_pci_device_id(const char* bus) {
    // hipDeviceGetPCIBusId gives "dddd:bb:dd.f"; sysfs holds the PCI device id as "0x75a3".
    char path[256];
    snprintf(path, sizeof path, "/sys/bus/pci/devices/%s/device", bus);
    for (char* p = path; *p; ++p) *p = char(std::tolower(*p));
    FILE* f = fopen(path, "r");
    if (!f) return 0;
    unsigned v = 0;
    if (fscanf(f, "%x", &v) != 1) v = 0;
    fclose(f);
    return v;
}

std::vector<DeviceInfo> Device::enumerate() {
    std::vector<DeviceInfo> out;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return out;
    }
    int rt = 0, drv = 0;
    (void)hipRuntimeGetVersion(&rt);
    (void)hipDriverGetVersion(&drv);
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) != hipSuccess) continue;
        DeviceInfo d{};
        d.index = i;
        snprintf(d.name, sizeof d.name, "%s", p.name);
        snprintf(d.arch, sizeof d.arch, "%s", p.gcnArchName);
        d.vendor_id = 0x1002;
        (void)hipDeviceGetPCIBusId(d.pci_bus, sizeof d.pci_bus, i);
        d.pci_device_id = read_pci_device_id(d.pci_bus);
        snprintf(d.driver, sizeof d.driver, "hip-runtime-%d/driver-%d", rt, drv);
        d.memory_bytes = int64_t(p.totalGlobalMem);
        d.compute_units = p.multiProcessorCount;
        out.push_back(d);
    }
    return out;
}

// ---------------------------------------------------------------- device

Device::Device(int index, uint32_t flags) : index_(index), flags_(flags) {
    auto all = enumerate();
    if (index < 0 || index >= int(all.size())) contract_fail("no HIP device %d (%zu found)", index, all.size());
    info_ = all[size_t(index)];
    HIPC(hipSetDevice(index));
    HIPC(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    HIPC(hipStreamCreateWithFlags(&side_, hipStreamNonBlocking));
    HIPC(hipEventCreateWithFlags(&fork_ev_, hipEventDisableTiming));
    HIPC(hipEventCreateWithFlags(&join_ev_, hipEventDisableTiming));
    HIPC(hipEventCreate(&epoch_));
    HIPC(hipEventRecord(epoch_, stream_));
    static_scratch_ = static_scratch_address(index);
    f16_range_[0] = f16_range_word_fast();
    f16_range_[1] = f16_range_word_persist();
}

uint32_t Device::take_f16_range() {
    HIPC(hipSetDevice(index_));
    uint32_t bits = 0;
    for (void* w : f16_range_) {
        uint32_t v = 0;
        HIPC(hipMemcpyAsync(&v, w, 4, hipMemcpyDeviceToHost, stream_));
        HIPC(hipStreamSynchronize(stream_));
        if (v) {
            const uint32_t zero = 0;
            HIPC(hipMemcpyAsync(w, &zero, 4, hipMemcpyHostToDevice, stream_));
            HIPC(hipStreamSynchronize(stream_));
        }
        bits |= v;
    }
    return bits;
}

std::string f16_range_sites(uint32_t bits) {
    static const char* names[] = {"normed hidden rows (h)", "query (q)", "K/V cache", "attention output (o)",
                                  "SwiGLU output (a)"};
    std::string out;
    for (int i = 0; i < 5; ++i)
        if (bits & (1u << i)) out += (out.empty() ? "" : ", ") + std::string(names[i]);
    return out;
}

Device::~Device() {
    (void)hipSetDevice(index_);
    (void)hipStreamSynchronize(stream_);
    for (auto& kv : pending_) {
        (void)hipEventDestroy(kv.second.done);
        for (auto& e : kv.second.timer_events) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
    }
    lists_.clear();
    for (void* p : pages_)
        if (p) (void)hipFree(p);
    for (auto& e : dispatch_events_) {
        (void)hipEventDestroy(e.first);
        (void)hipEventDestroy(e.second);
    }
    if (epoch_) (void)hipEventDestroy(epoch_);
    if (fork_ev_) (void)hipEventDestroy(fork_ev_);
    if (join_ev_) (void)hipEventDestroy(join_ev_);
    if (side_) (void)hipStreamDestroy(side_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

void Device::create_heap(const HeapLayout& layout) {
    if (heap_created_) contract_fail("CreateHeap runs exactly once per backend");
    HIPC(hipSetDevice(index_));
    layout_ = layout;
    pages_.assign(size_t(kSlotCount), nullptr);
    HIPC(hipMalloc(&pages_[0], kTableBytes));
    HIPC(hipMemsetAsync(pages_[0], 0, kTableBytes, stream_));
    for (const Page& p : layout.pages) {
        HIPC(hipMalloc(&pages_[size_t(p.slot)], p.bytes));
        HIPC(hipMemsetAsync(pages_[size_t(p.slot)], 0, p.bytes, stream_));
    }
    HIPC(hipStreamSynchronize(stream_));
    heap_created_ = true;
}

const HeapLayout& Device::layout() const {
    if (!heap_created_) contract_fail("the heap has not been created");
    return layout_;
}

void Device::write_table(const void* image, uint64_t bytes) {
    if (!heap_created_) contract_fail("WriteTable needs the heap");
    if (!table_host_.empty()) contract_fail("WriteTable runs exactly once, before the first dispatch");
    if (bytes != kTableBytes) contract_fail("a table image is %llu bytes, not 1 MiB", (unsigned long long)kTableBytes);
    const uint8_t* img = static_cast<const uint8_t*>(image);
    SealedTableView v{img};
    if (!v.row(0).is_zero()) contract_fail("row 0 of the table is the null row and must be zero");
    for (uint32_t t = 1; t < uint32_t(kTableRows); ++t) {
        TensorRow r = v.row(t);
        if (r.is_zero()) continue;
        try {
            r.validate(layout_);
        } catch (const ContractError& e) {
            contract_fail("table row %u: %s", t, e.what());
        }
    }
    HIPC(hipStreamSynchronize(stream_));
    HIPC(hipMemcpy(pages_[0], image, kTableBytes, hipMemcpyHostToDevice));
    table_host_.assign(img, img + kTableBytes);
}

SealedTableView Device::table() const {
    if (table_host_.empty()) contract_fail("the table has not been written");
    return SealedTableView{table_host_.data()};
}

void Device::upload(int slot, uint64_t offset, const void* src, uint64_t bytes) {
    if (!heap_created_) contract_fail("Upload needs the heap");
    check_transfer(layout_, slot, offset, bytes, false);
    HIPC(hipStreamSynchronize(stream_));
    const uint8_t* s = static_cast<const uint8_t*>(src);
    const uint64_t chunk = 64ull << 20;  // UploadFrom stages in chunks of at most 64 MiB
    for (uint64_t done = 0; done < bytes; done += chunk) {
        uint64_t n = bytes - done < chunk ? bytes - done : chunk;
        HIPC(hipMemcpy(static_cast<uint8_t*>(pages_[size_t(slot)]) + offset + done, s + done, n, hipMemcpyHostToDevice));
    }
}

void Device::download(int slot, uint64_t offset, void* dst, uint64_t bytes) {
    if (!heap_created_) contract_fail("Download needs the heap");
    check_transfer(layout_, slot, offset, bytes, true);
    HIPC(hipStreamSynchronize(stream_));
    HIPC(hipMemcpy(dst, static_cast<uint8_t*>(pages_[size_t(slot)]) + offset, bytes, hipMemcpyDeviceToHost));
}

void* Device::slot_ptr(int slot) const {
    if (slot < 0 || slot >= int(pages_.size()) || !pages_[size_t(slot)]) contract_fail("slot %d holds no buffer", slot);
    return pages_[size_t(slot)];
}

void* Device::resolve(uint32_t token) const {
    TensorRow r = table().row(token);
    return static_cast<uint8_t*>(slot_ptr(int(r.slot()))) + r.offset();
}

// ---------------------------------------------------------------- kernels

static std::array<uint8_t, 32> hash_of_this_library() {
    Dl_info dl{};
    std::array<uint8_t, 32> zero{};
    if (!dladdr(reinterpret_cast<void*>(&hash_of_this_library), &dl) || !dl.dli_fname) return zero;
    std::ifstream f(dl.dli_fname, std::ios::binary);
    if (!f) return zero;
    std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    return Sha256::of(bytes.data(), bytes.size());
}

std::array<uint8_t, 32> Device::load_kernels(KernelSet set) {
    if (loaded_) contract_fail("LoadKernels runs exactly once per backend");
    if (set != KernelSet::Reference && set != KernelSet::Fast) contract_fail("unknown kernel set %d", int(set));
    HIPC(hipSetDevice(index_));
    const std::array<uint8_t, 32> lib = hash_of_this_library();
    std::string msg = set == KernelSet::Reference ? "lrm-hip kernel set: reference\n" : "lrm-hip kernel set: fast\n";
    msg.append(reinterpret_cast<const char*>(lib.data()), lib.size());
    shader_hash_ = Sha256::of(msg.data(), msg.size());
    set_ = set;
    loaded_ = true;
    run_probe();
    return shader_hash_;
}

bool Device::contains(int kernel) const {
    if (kernel < 0 || kernel >= catalog_size()) return false;
    if (set_ == KernelSet::Reference && kernel >= fast_first_id()) return false;
    if (kernel < fast_first_id()) return catalog_launchers()[kernel] != nullptr;
    return fast_launchers()[kernel - fast_first_id()] != nullptr;
}

static LaunchFn launcher_of(int kernel) {
    return kernel < fast_first_id() ? catalog_launchers()[kernel] : fast_launchers()[kernel - fast_first_id()];
}

// The fp32 denormal probe (gpu-backend.md "fp32 denormals"; Backend.fs:457-547): scale_f32 with a = 0.5 over seven
// inputs; Preserve when the bits equal the CPU's, Flush when they equal the CPU's with denormals replaced by zero.
void Device::run_probe() {
    static const uint32_t in[7] = {0x3f800000u, 0x01000000u, 0x00800000u, 0x80800000u,
                                   0x00000002u, 0x807ffffeu, 0x00400000u};
    static const uint32_t preserve[7] = {0x3f000000u, 0x00800000u, 0x00400000u, 0x80400000u,
                                         0x00000001u, 0x803fffffu, 0x00200000u};
    static const uint32_t flush[7] = {0x3f000000u, 0x00800000u, 0x00000000u, 0x80000000u,
                                      0x00000000u, 0x80000000u, 0x00000000u};
    void* buf = nullptr;
    HIPC(hipMalloc(&buf, 64));
    HIPC(hipMemcpy(buf, in, sizeof in, hipMemcpyHostToDevice));
    PreparedDispatch pd{};
    pd.kernel = catalog_find("scale_f32");
    uint32_t half;
    float h = 0.5f;
    std::memcpy(&half, &h, 4);
    pd.words = {};
    pd.words[0] = 1;
    pd.words[3] = 7;
    pd.words[4] = half;
    pd.physical = Physical{1, 1, 1};
    pd.grid = Grid3{1, 1, 1};
    void* ptr[4] = {buf, static_cast<uint8_t*>(buf) + 32, nullptr, nullptr};
    launcher_of(pd.kernel)(pd, ptr, stream_);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(stream_));
    HIPC(hipMemcpy(probe_results_.data(), static_cast<uint8_t*>(buf) + 32, 28, hipMemcpyDeviceToHost));
    HIPC(hipFree(buf));
    bool is_p = std::memcmp(probe_results_.data(), preserve, 28) == 0;
    bool is_f = std::memcmp(probe_results_.data(), flush, 28) == 0;
    if (probe_results_[0] != preserve[0] || probe_results_[1] != preserve[1])
        contract_fail("the denormal probe's normal controls are wrong: scale_f32 itself failed");
    denormal_mode_ = is_p ? 1 : is_f ? 2 : 3;
}

// ---------------------------------------------------------------- command lists

CommandList::~CommandList() {
    if (exec_) (void)hipGraphExecDestroy(exec_);
    if (graph_) (void)hipGraphDestroy(graph_);
}

void CommandList::check_open() const {
    if (closed_) contract_fail("a command list is used once: Submit closed it");
}

void CommandList::dispatch(int kernel, const uint32_t* words) {
    check_open();
    if (exec_) contract_fail("a reusable list cannot be changed after its first submission");
    if (!dev_->kernels_loaded()) contract_fail("Dispatch before LoadKernels");
    if (!dev_->contains(kernel)) contract_fail("kernel %d is not in the loaded kernel set", kernel);
    Cmd c{};
    c.kind = Cmd::Launch;
    c.pd = prepare(dev_->table(), kernel, words);
    const KernelSpec& k = catalog()[size_t(kernel)];
    c.ptr.assign(k.fields.size() + 1, nullptr);
    for (const TokenUse& u : c.pd.tokens) {
        if (u.access == Access::Meta)
            c.ptr[size_t(u.field)] = static_cast<uint8_t*>(dev_->slot_ptr(0)) + size_t(u.token) * kRowBytes;
        else
            c.ptr[size_t(u.field)] = dev_->resolve(u.token);
    }
    cmds_.push_back(std::move(c));
    ++dispatches_;
}

void CommandList::dispatch_library(int kernel, const uint32_t* words, int library_field, void* library_ptr) {
    const LibraryDispatch d{kernel, words, library_field, library_ptr};
    dispatch_library_all(&d, 1, nullptr);
}

void CommandList::dispatch_library_all(const LibraryDispatch* d, size_t n, const LibraryCheck& check) {
    check_open();
    if (exec_) contract_fail("a reusable list cannot be changed after its first submission");
    if (!dev_->kernels_loaded()) contract_fail("Dispatch before LoadKernels");
    std::vector<Cmd> staged;
    staged.reserve(n);
    for (size_t i = 0; i < n; ++i) {
        if (!dev_->contains(d[i].kernel)) contract_fail("kernel %d is not in the loaded kernel set", d[i].kernel);
        if (!d[i].library_ptr) contract_fail("no library buffer for field %d", d[i].library_field);
        Cmd c{};
        c.kind = Cmd::Launch;
        c.pd = prepare_library_field(dev_->table(), d[i].kernel, d[i].words, d[i].library_field);
        const KernelSpec& k = catalog()[size_t(d[i].kernel)];
        c.ptr.assign(k.fields.size() + 1, nullptr);
        for (const TokenUse& u : c.pd.tokens) {
            if (u.access == Access::Meta)
                c.ptr[size_t(u.field)] = static_cast<uint8_t*>(dev_->slot_ptr(0)) + size_t(u.token) * kRowBytes;
            else
                c.ptr[size_t(u.field)] = dev_->resolve(u.token);
        }
        c.ptr[size_t(d[i].library_field)] = d[i].library_ptr;
        staged.push_back(std::move(c));
    }
    if (check) {
        std::vector<const PreparedDispatch*> pds;
        for (const Cmd& c : staged) pds.push_back(&c.pd);
        check(pds);
    }
    // nothing was refused: record them all
    for (Cmd& c : staged) {
        cmds_.push_back(std::move(c));
        ++dispatches_;
    }
}

void CommandList::dispatch_overlapped(int kernel, const uint32_t* words) {
    dispatch(kernel, words);
    cmds_.back().kind = Cmd::LaunchSide;
    side_open_ = true;
}

void CommandList::barrier() {
    check_open();
    // The main stream is in order: every earlier command on it has finished its writes before a later one starts.
    // Overlapped dispatches are joined here.
    if (side_open_) {
        if (exec_) contract_fail("a reusable list cannot be changed after its first submission");
        Cmd c{};
        c.kind = Cmd::Join;
        cmds_.push_back(std::move(c));
        side_open_ = false;
    }
}

void CommandList::copy(int ss, uint64_t so, int ds, uint64_t dof, uint64_t bytes) {
    check_open();
    if (exec_) contract_fail("a reusable list cannot be changed after its first submission");
    check_copy(dev_->layout(), ss, so, ds, dof, bytes);
    Cmd c{};
    c.kind = Cmd::Copy;
    c.src = static_cast<uint8_t*>(dev_->slot_ptr(ss)) + so;
    c.dst = static_cast<uint8_t*>(dev_->slot_ptr(ds)) + dof;
    c.bytes = bytes;
    cmds_.push_back(std::move(c));
}

int CommandList::begin_timer(const std::string& name) {
    check_open();
    if (name.empty()) contract_fail("a timer needs a telemetry name");
    int id = int(timer_names_.size());
    timer_names_.push_back(name);
    open_timers_.push_back(id);
    Cmd c{};
    c.kind = Cmd::TimerBegin;
    c.timer = id;
    cmds_.push_back(std::move(c));
    return id;
}

void CommandList::end_timer(int timer) {
    check_open();
    if (open_timers_.empty() || open_timers_.back() != timer)
        contract_fail("timers close in reverse order of opening (closing %d)", timer);
    open_timers_.pop_back();
    Cmd c{};
    c.kind = Cmd::TimerEnd;
    c.timer = timer;
    cmds_.push_back(std::move(c));
}

CommandList* Device::begin(bool reusable) {
    lists_.emplace_back(new CommandList(this, reusable));
    return lists_.back().get();
}

void Device::release(CommandList* l) {
    for (auto it = lists_.begin(); it != lists_.end(); ++it)
        if (it->get() == l) {
            lists_.erase(it);
            return;
        }
}

// Reusable lists replay as HIP graphs unless LRM_HIP_GRAPHS=0 (for tools that cannot trace stream capture).
bool Device::graphs_enabled() {
    static const bool on = [] {
        const char* v = std::getenv("LRM_HIP_GRAPHS");
        return !(v && v[0] == '0');
    }();
    return on;
}

void Device::launch_side(const CommandList::Cmd& c) {
    HIPC(hipEventRecord(fork_ev_, stream_));
    HIPC(hipStreamWaitEvent(side_, fork_ev_, 0));
    launcher_of(c.pd.kernel)(c.pd, c.ptr.data(), side_);
}

void Device::join_side() {
    HIPC(hipEventRecord(join_ev_, side_));
    HIPC(hipStreamWaitEvent(stream_, join_ev_, 0));
}

void Device::run(CommandList* l) {
    bool side = false;
    for (auto& c : l->cmds_) {
        if (c.kind == CommandList::Cmd::Launch) {
            launcher_of(c.pd.kernel)(c.pd, c.ptr.data(), stream_);
        } else if (c.kind == CommandList::Cmd::LaunchSide) {
            launch_side(c);
            side = true;
        } else if (c.kind == CommandList::Cmd::Join) {
            join_side();
            side = false;
        } else if (c.kind == CommandList::Cmd::Copy) {
            HIPC(hipMemcpyAsync(c.dst, c.src, c.bytes, hipMemcpyDeviceToDevice, stream_));
        }
    }
    if (side) join_side();  // the list ends with every overlapped dispatch joined (and, under capture, in the graph)
}

uint64_t Device::submit(CommandList* l, uint32_t repeat) {
    bool mine = false;
    for (auto& p : lists_) mine = mine || p.get() == l;
    if (!mine) contract_fail("the command list belongs to another backend or was released");
    l->check_open();
    if (!l->open_timers_.empty()) contract_fail("a command list cannot be submitted with a timer open");
    if (repeat < 1) contract_fail("a submission runs its list at least once");
    if (repeat > 1 && !l->reusable_) contract_fail("only a reusable list can be replayed");
    HIPC(hipSetDevice(index_));
    Pending pend{};
    pend.dispatches = l->dispatches_ * int(repeat);
    pend.owned = nullptr;
    if (!l->reusable_) {
        // One-shot: launch every command now, with timer events and per-dispatch timing as asked.
        std::vector<std::pair<hipEvent_t, hipEvent_t>> tev(l->timer_names_.size());
        bool time_dispatches = (flags_ & TimeDispatches) != 0;
        bool side = false;
        for (auto& c : l->cmds_) {
            switch (c.kind) {
                case CommandList::Cmd::Launch: {
                    hipEvent_t a = nullptr, b = nullptr;
                    if (time_dispatches) {
                        HIPC(hipEventCreate(&a));
                        HIPC(hipEventCreate(&b));
                        HIPC(hipEventRecord(a, stream_));
                    }
                    launcher_of(c.pd.kernel)(c.pd, c.ptr.data(), stream_);
                    HIPC(hipGetLastError());
                    if (time_dispatches) {
                        HIPC(hipEventRecord(b, stream_));
                        pend.timer_events.emplace_back(a, b);
                        pend.timer_names.push_back(std::string("gpu.dispatch/") + catalog()[size_t(c.pd.kernel)].name);
                    }
                    break;
                }
                case CommandList::Cmd::LaunchSide:
                    launch_side(c);
                    side = true;
                    break;
                case CommandList::Cmd::Join:
                    join_side();
                    side = false;
                    break;
                case CommandList::Cmd::Copy:
                    HIPC(hipMemcpyAsync(c.dst, c.src, c.bytes, hipMemcpyDeviceToDevice, stream_));
                    break;
                case CommandList::Cmd::TimerBegin:
                    HIPC(hipEventCreate(&tev[size_t(c.timer)].first));
                    HIPC(hipEventRecord(tev[size_t(c.timer)].first, stream_));
                    break;
                case CommandList::Cmd::TimerEnd:
                    HIPC(hipEventCreate(&tev[size_t(c.timer)].second));
                    HIPC(hipEventRecord(tev[size_t(c.timer)].second, stream_));
                    break;
            }
        }
        if (side) join_side();
        // Timers first, in the order opened, then the dispatch timings (Completion.Timers).
        std::vector<std::pair<hipEvent_t, hipEvent_t>> all(tev.begin(), tev.end());
        std::vector<std::string> names(l->timer_names_.begin(), l->timer_names_.end());
        all.insert(all.end(), pend.timer_events.begin(), pend.timer_events.end());
        names.insert(names.end(), pend.timer_names.begin(), pend.timer_names.end());
        pend.timer_events = all;
        pend.timer_names = names;
        l->closed_ = true;
        pend.owned = l;
    } else if (!graphs_enabled()) {
        // Profilers that cannot follow stream capture: replay by launching the recorded commands directly.
        if (!l->timer_names_.empty()) contract_fail("a reusable list cannot hold timers");
        for (uint32_t r = 0; r < repeat; ++r) run(l);
        HIPC(hipGetLastError());
    } else {
        if (!l->timer_names_.empty()) contract_fail("a reusable list cannot hold timers");
        if (!l->exec_) {
            HIPC(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
            try {
                run(l);
            } catch (...) {
                hipGraph_t g = nullptr;
                (void)hipStreamEndCapture(stream_, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            HIPC(hipStreamEndCapture(stream_, &l->graph_));
            HIPC(hipGraphInstantiate(&l->exec_, l->graph_, nullptr, nullptr, 0));
        }
        for (uint32_t r = 0; r < repeat; ++r) HIPC(hipGraphLaunch(l->exec_, stream_));
    }
    HIPC(hipEventCreate(&pend.done));
    HIPC(hipEventRecord(pend.done, stream_));
    uint64_t fence = next_fence_++;
    pending_[fence] = std::move(pend);
    return fence;
}

const Completion& Device::wait(uint64_t fence) {
    auto d = done_.find(fence);
    if (d != done_.end()) return d->second;
    auto it = pending_.find(fence);
    if (it == pending_.end()) {
        if (fence >= 1 && fence < next_fence_)
            contract_fail("submission %llu completed and its completion was dropped: the backend keeps the last %zu",
                          (unsigned long long)fence, kKeptCompletions);
        contract_fail("submission %llu was never made on this backend", (unsigned long long)fence);
    }
    Pending& p = it->second;
    hipError_t e = hipEventSynchronize(p.done);
    if (e != hipSuccess) {
        hip_check(e, "waiting for a submission (device lost or a kernel faulted)");
    }
    Completion c;
    c.submission = fence;
    c.dispatches = p.dispatches;
    for (size_t i = 0; i < p.timer_events.size(); ++i) {
        float start = 0.f, dur = 0.f;
        HIPC(hipEventElapsedTime(&start, epoch_, p.timer_events[i].first));
        HIPC(hipEventElapsedTime(&dur, p.timer_events[i].first, p.timer_events[i].second));
        c.timers.push_back(TimerResult{p.timer_names[i], int64_t(double(start) * 1e6), int64_t(double(dur) * 1e6)});
        (void)hipEventDestroy(p.timer_events[i].first);
        (void)hipEventDestroy(p.timer_events[i].second);
    }
    (void)hipEventDestroy(p.done);
    pending_.erase(it);
    // Waiting again returns the same completion (gpu-backend.md, IGpuBackend.Wait), for the most recent
    // kKeptCompletions submissions waited on; older ones are dropped, so a decode loop that submits and waits once per
    // token holds bounded host memory.
    while (done_.size() >= kKeptCompletions) done_.erase(done_.begin());
    return done_.emplace(fence, std::move(c)).first->second;
}

}  // namespace lrm
