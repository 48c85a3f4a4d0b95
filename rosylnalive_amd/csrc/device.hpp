// The HIP device behind the reference's Lrm.Gpu.Core interfaces (src/Lrm.Gpu.Core/Backend.fs:104-161):
// IGpuBackend (Device), IGpuHeap (the heap methods of Device), ICommandList (CommandList), IKernelSet (load/contains).
//
// MI355X-first choices, all invisible to callers of the contract:
//   - one in-order HIP stream per device, so Barrier() costs nothing and Copy() is ordered on both sides;
//   - the sealed table is kept on the host too: every token is resolved to a device pointer when a dispatch is
//     recorded, and kernels receive plain pointers and the scalar argument words;
//   - a fence is a hipEvent recorded after a submission; Wait synchronises it and returns the stored Completion;
//   - a command list created reusable is captured into a hipGraph at its first submission and replayed by every later
//     submission (the decode step of the executor): zero host work per replay.
#pragma once

#include <hip/hip_runtime_api.h>

#include <array>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "contract.hpp"

namespace lrm {

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// A value the fast path stores as fp16 (an activation or a K/V cache entry) became inf or NaN: the call's results
// are not usable.
struct RangeError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void hip_check(hipError_t e, const char* what);

// The launch function of one catalog kernel: pointers per field (nullptr for non-token fields), the prepared words.
using LaunchFn = void (*)(const PreparedDispatch& pd, void* const* ptr, hipStream_t stream);
// One table per kernel source file; entry i is catalog id i or nullptr.
const LaunchFn* catalog_launchers();  // ids 0..13
const LaunchFn* fast_launchers();     // ids 14..
int fast_first_id();

class Device;
class CommandList;
// The library's static scratch (scratch_static.hip): its size, this GPU's copy (hipGetSymbolAddress with `device`
// current, looked up once per device), and the decode attention whose split partials live there.
size_t static_scratch_bytes();
void* static_scratch_address(int device);
void record_decode_attention_static(Device& dev, CommandList* l, const uint32_t* words, uint32_t y);
// The fp16 range words of the fast-path and persistent-decode code objects on the current GPU (hipGetSymbolAddress):
// sticky bits of the sites where a kernel stored an inf or NaN half (1 normed hidden rows, 2 q, 4 K/V cache, 8 attention
// output, 16 SwiGLU output).
void* f16_range_word_fast();
bool gemm_stamps_read(int kind, uint64_t* dst, size_t words);  // kernels_fast.hip: the stage-timing build's stamps
void* f16_range_word_persist();
// The site names of a set of those bits, comma-separated.
std::string f16_range_sites(uint32_t bits);
constexpr uint32_t kF16SiteSwiglu = 16u;  // the SwiGLU output's bit in that word

struct DeviceInfo {
    int index;
    char name[128];
    char arch[64];
    uint32_t vendor_id;
    uint32_t pci_device_id;
    char pci_bus[32];
    char driver[64];
    int64_t memory_bytes;
    int compute_units;
};

struct TimerResult {
    std::string name;
    int64_t start_ns;
    int64_t duration_ns;
};

struct Completion {
    uint64_t submission;
    int dispatches;
    std::vector<TimerResult> timers;
};

class Device;

class CommandList {
  public:
    void dispatch(int kernel, const uint32_t* words);
    // A dispatch that may run concurrently with the dispatches after it, up to the next barrier (the reference's
    // ordering rule: dispatches not separated by Barrier may overlap). It runs on the device's side stream, after
    // everything recorded before it; Barrier, and the end of the list, wait for it.
    void dispatch_overlapped(int kernel, const uint32_t* words);
    // A dispatch whose token field `library_field` is device memory the library owns (`library_ptr`) rather than a
    // tensor of the heap; its word is 0 (prepare_library_field). The caller has checked the bytes the launch touches.
    void dispatch_library(int kernel, const uint32_t* words, int library_field, void* library_ptr);
    // Several library dispatches recorded together or not at all: each is prepared (every contract check) before the
    // first is recorded, and `check`, when set, sees their prepared argument words and may refuse the group by
    // throwing. A refused group leaves the list as it was.
    struct LibraryDispatch {
        int kernel;
        const uint32_t* words;
        int library_field;
        void* library_ptr;
    };
    using LibraryCheck = std::function<void(const std::vector<const PreparedDispatch*>&)>;
    void dispatch_library_all(const LibraryDispatch* d, size_t n, const LibraryCheck& check);
    void barrier();
    void copy(int src_slot, uint64_t src_off, int dst_slot, uint64_t dst_off, uint64_t bytes);
    int begin_timer(const std::string& name);
    void end_timer(int timer);
    int dispatch_count() const { return dispatches_; }
    bool reusable() const { return reusable_; }
    ~CommandList();

  private:
    friend class Device;
    struct Cmd {
        enum Kind { Launch, LaunchSide, Join, Copy, TimerBegin, TimerEnd } kind;
        PreparedDispatch pd;
        std::vector<void*> ptr;
        void* src = nullptr;
        void* dst = nullptr;
        uint64_t bytes = 0;
        int timer = -1;
    };
    CommandList(Device* d, bool reusable) : dev_(d), reusable_(reusable) {}
    void check_open() const;
    Device* dev_;
    bool reusable_;
    bool closed_ = false;      // a one-shot list after Submit
    std::vector<Cmd> cmds_;
    std::vector<std::string> timer_names_;
    std::vector<int> open_timers_;
    int dispatches_ = 0;
    bool side_open_ = false;  // an overlapped dispatch not yet joined
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
};

class Device {
  public:
    enum Flags : uint32_t { TimeDispatches = 1 };
    static std::vector<DeviceInfo> enumerate();
    Device(int index, uint32_t flags);
    ~Device();

    const DeviceInfo& info() const { return info_; }

    // IGpuHeap
    void create_heap(const HeapLayout& layout);
    void write_table(const void* image, uint64_t bytes);
    void upload(int slot, uint64_t offset, const void* src, uint64_t bytes);
    void download(int slot, uint64_t offset, void* dst, uint64_t bytes);
    const HeapLayout& layout() const;
    bool table_written() const { return !table_host_.empty(); }
    SealedTableView table() const;

    // IKernelSet. Two kernel sets, each its own ExecutionClass (its own shader-set hash), since they make different
    // bit-identity claims:
    //   Reference: the reference's catalog, ids 0 .. fast_first_id() - 1, which keeps the BatchInvariance contract
    //     (a row alone equals the row in any batch; prefill equals decode and any chunked prefill);
    //   Fast: every id (the reference's catalog and the fast path), which only claims that the same work on the same
    //     inputs gives the same bits: its k-split and attention-split choices depend on the row count, and its
    //     prefill and decode kernels sum in different orders.
    // The hash is the SHA-256 of the set's name and the library file's SHA-256.
    enum class KernelSet { Reference = 0, Fast = 1 };
    std::array<uint8_t, 32> load_kernels(KernelSet set = KernelSet::Reference);
    bool kernels_loaded() const { return loaded_; }
    KernelSet kernel_set() const { return set_; }
    bool contains(int kernel) const;
    const std::array<uint8_t, 32>& shader_set_hash() const { return shader_hash_; }
    // fp32 denormal mode measured by the probe after load_kernels (gpu-backend.md "fp32 denormals"): 0 unknown,
    // 1 preserve, 2 flush, 3 mixed.
    int denormal_mode() const { return denormal_mode_; }
    const std::array<uint32_t, 7>& denormal_results() const { return probe_results_; }

    // IGpuBackend
    CommandList* begin(bool reusable = false);
    uint64_t submit(CommandList* list, uint32_t repeat = 1);
    const Completion& wait(uint64_t fence);
    void release(CommandList* list);  // frees a list; the caller releases every list it began

    hipStream_t stream() const { return stream_; }
    int index() const { return index_; }
    // This device's copy of the library's static scratch array (its address from hipGetSymbolAddress at creation)
    void* static_scratch() const { return static_scratch_; }
    // The fp16 range sites (bits as f16_range_word_fast) that kernels on this GPU flagged since the last call, then
    // cleared. The words are per GPU, shared by every backend on it; call after the work in question has completed.
    uint32_t take_f16_range();
    void* slot_ptr(int slot) const;
    void* resolve(uint32_t token) const;  // device pointer of a token's first byte

  private:
    friend class CommandList;
    void run(CommandList* l);
    void launch_side(const CommandList::Cmd& c);  // fork from the main stream, launch on the side stream
    void join_side();                             // the main stream waits for the side stream
    static bool graphs_enabled();
    void run_probe();
    DeviceInfo info_{};
    int index_;
    uint32_t flags_;
    hipStream_t stream_ = nullptr;
    hipStream_t side_ = nullptr;  // overlapped dispatches (default priority, like stream_)
    hipEvent_t fork_ev_ = nullptr, join_ev_ = nullptr;
    hipEvent_t epoch_ = nullptr;
    void* static_scratch_ = nullptr;
    void* f16_range_[2] = {nullptr, nullptr};
    bool heap_created_ = false;
    HeapLayout layout_;
    std::vector<void*> pages_;  // slot i at pages_[i], slot 0 = the table buffer
    std::vector<uint8_t> table_host_;
    bool loaded_ = false;
    KernelSet set_ = KernelSet::Reference;
    std::array<uint8_t, 32> shader_hash_{};
    int denormal_mode_ = 0;
    std::array<uint32_t, 7> probe_results_{};
    uint64_t next_fence_ = 1;
    struct Pending {
        hipEvent_t done;
        std::vector<std::pair<hipEvent_t, hipEvent_t>> timer_events;
        std::vector<std::string> timer_names;
        int dispatches;
        CommandList* owned;  // one-shot list to free after completion
    };
    std::map<uint64_t, Pending> pending_;
    std::map<uint64_t, Completion> done_;  // the last kKeptCompletions waited on, by fence

  public:
    static constexpr size_t kKeptCompletions = 1024;

  private:
    std::vector<std::unique_ptr<CommandList>> lists_;
    // dispatch timing (TimeDispatches)
    std::vector<std::pair<hipEvent_t, hipEvent_t>> dispatch_events_;
};

}  // namespace lrm
