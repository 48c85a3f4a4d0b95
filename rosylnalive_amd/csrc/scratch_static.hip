// The library's static scratch: one file-scope device array that each GPU holds from the library's load until the
// process ends, so a caller that cannot allocate device memory (code under HIP graph capture, serving loops that
// forbid allocation) can still run the kernels that need scratch beyond their inputs and outputs.
//
// The array's name is a host-side stand-in, not a device address: host code never passes it to a kernel, a copy or a
// memset. Each Device looks up its own GPU's copy once, at creation, with hipGetSymbolAddress (with that device
// current) and passes that pointer as the kernels' argument.
//
// Every call on one GPU shares that GPU's array, which keeps the last call's contents: calls that may overlap on one
// GPU (lists submitted from two backends of the same GPU) race. Nothing here needs the array to start at zero: the
// decode attention writes every partial row its combine reads.
#include <hip/hip_runtime.h>

#include <mutex>

#include "device.hpp"

static constexpr size_t kStaticScratchBytes = size_t(4) << 20;
static __device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];

namespace lrm {

size_t static_scratch_bytes() { return kStaticScratchBytes; }

void* static_scratch_address(int device) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) contract_fail("static scratch: device index %d", device);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {
        int cur = -1;
        hip_check(hipGetDevice(&cur), "hipGetDevice");
        if (cur != device) contract_fail("static scratch: device %d is not current (%d is)", device, cur);
        void* p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p) throw HipError("hipGetSymbolAddress(scratch) returned a null address");
        addr[device] = p;
    }
    return addr[device];
}

// attention_decode_f16 then attention_combine (f32 output), the split partials in this GPU's static scratch.
// words: the attention_decode_f16 argument block with its partials word 0; y: the combine's output token.
// Both dispatches are contract-checked, and the partials' bytes are computed from the checked words, before either
// is recorded: a refused call leaves the list unchanged.
void record_decode_attention_static(Device& dev, CommandList* l, const uint32_t* words, uint32_t y) {
    const int dec = catalog_find("attention_decode_f16"), comb = catalog_find("attention_combine");
    uint32_t cw[32] = {0};
    cw[2] = y;              // y
    cw[3] = words[9];       // state
    cw[4] = words[10];      // q_heads
    cw[5] = words[12];      // max_pos
    cw[6] = words[15];      // batch
    cw[7] = words[16];      // chunks
    cw[8] = words[17];      // splits
    void* p = dev.static_scratch();
    const CommandList::LibraryDispatch both[2] = {{dec, words, 7, p}, {comb, cw, 0, p}};
    l->dispatch_library_all(both, 2, [](const std::vector<const PreparedDispatch*>& pd) {
        // the bytes the launches touch: per sequence and query head, one 130-float row per split
        const uint32_t* w = pd[0]->words.data();
        const uint64_t qh = w[10], mp = w[12], B = w[15], chunks = w[16] ? w[16] : 1, splits = w[17];
        const uint64_t S = splits ? splits : (mp + 64 * chunks - 1) / (64 * chunks);
        const uint64_t bytes = B * qh * S * 130 * sizeof(float);
        if (bytes > kStaticScratchBytes)
            contract_fail("decode attention (static scratch): %llu sequences x %llu query heads x %llu splits need "
                          "%llu bytes of split partials; the static scratch holds %zu",
                          (unsigned long long)B, (unsigned long long)qh, (unsigned long long)S,
                          (unsigned long long)bytes, kStaticScratchBytes);
    });
}

}  // namespace lrm
