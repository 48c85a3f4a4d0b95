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

uint32_t decode_attention_splits(uint32_t max_pos, uint32_t chunks, uint32_t splits);  // kernels_fast.hip

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
void record_decode_attention_static(Device& dev, CommandList* l, const uint32_t* words, uint32_t y) {
    const int dec = catalog_find("attention_decode_f16"), comb = catalog_find("attention_combine");
    const uint32_t qh = words[10], mp = words[12], B = words[15], chunks = words[16], splits = words[17];
    // the bytes the launches touch: per sequence and query head, one 130-float row per split
    const uint64_t S = decode_attention_splits(mp, chunks, splits);
    const uint64_t bytes = uint64_t(B) * qh * S * 130 * sizeof(float);
    if (bytes > kStaticScratchBytes)
        contract_fail("decode attention (static scratch): %u sequences x %u query heads x %llu splits need %llu bytes "
                      "of split partials; the static scratch holds %zu",
                      B, qh, (unsigned long long)S, (unsigned long long)bytes, kStaticScratchBytes);
    void* p = dev.static_scratch();
    l->dispatch_library(dec, words, 7, p);
    uint32_t cw[32] = {0};
    cw[2] = y;            // y
    cw[3] = words[9];     // state
    cw[4] = qh;           // q_heads
    cw[5] = mp;           // max_pos
    cw[6] = B;            // batch
    cw[7] = chunks;       // chunks
    cw[8] = splits;       // splits
    l->dispatch_library(comb, cw, 0, p);
}

}  // namespace lrm
