// Shapes and exchange layout of the persistent one-sequence decode step (kernels_persist.hip), shared by the kernel,
// its launcher and the executor that sizes its buffers.
#pragma once

#include <cstdint>

namespace lrm {
namespace persist {

constexpr int kWaves = 8, kThreads = 512;
// Header before the entries: u32 word 0 = launch epoch, 1 = abort, 2 = the stage that aborted, 3 = the bound of every
// wait in 100 MHz constant-clock ticks (0: 0.2 s); words kClaimWord .. + 255: the role claims, one per (XCD, j), each
// holding the tag of the last launch whose workgroup took that role (a second claim in one launch aborts the step).
constexpr int kHdrEntries = 32 + 128;
constexpr int kClaimWord = 64;
constexpr int kStageClaim = 9;  // the abort stage of a role taken twice
constexpr int kVecMax = 8704;  // floats of the LDS vector a stage gathers its input into
// The accelerator complex dies (XCDs) of an MI355X, each with its own L2. KV head h lives on XCD h: its q|k|v rows,
// attention splits, and the o_proj / down_proj columns that read them, so three of a layer's five hand-offs stay
// inside one L2.
constexpr int kXcds = 8;
// 4-byte entries per (query head, split) attention partial row: out[128], max, sum, padded to whole 128-byte lines, so
// one wave writes every line of a row whole (lines written in part by several waves cost a read-modify-write each).
// The first kPartVecs 16-byte vectors (out, max, sum, two pad entries) are what the readers poll.
constexpr int kPartStride = 160, kPartVecs = 33;

struct Shape {
    int hidden, heads, kv_heads, head_dim, inter, max_pos, blocks;
};

// The exchange area, per layer:
//   8-byte entries (tag << 32) | value bits, one block per XCD (4 KB aligned, so no cache line is written by two
//   XCDs): the XCD's q|k|v rows (its query heads, key, value: 128 each);
//   4-byte entries, the value with its lowest mantissa bit replaced by the launch parity: one block per XCD holding
//   its attention partials per (query head, split) in rows of kPartStride entries and its slice of the SwiGLU output
//   (inter / kXcds), then the device-wide partial sums [kXcds][hidden] of o_proj (p1) and of down_proj (p2), each XCD's
//   columns summed alone.
// The XCD blocks are written and read by one XCD only; p1, p2, the lm_head partials and the header by all.
struct XLayout {
    int qkv, blk64, per_layer64;             // 8-byte entries
    int part, a, blk32, p1, p2, per_layer32;  // 4-byte entries
#if defined(__HIPCC__)
    __host__ __device__
#endif
    XLayout(int qh, int kvh, int hidden, int inter, int blocks) {
        const int S = blocks / kXcds, qpk = qh / kvh;
        qkv = 0;
        blk64 = ((qpk + 2) * 128 + 511) / 512 * 512;
        per_layer64 = kXcds * blk64;
        part = 0;
        a = qpk * S * kPartStride;
        blk32 = (a + inter / kXcds + 1023) / 1024 * 1024;
        p1 = kXcds * blk32;
        p2 = p1 + kXcds * hidden;
        per_layer32 = (p2 + kXcds * hidden + 1023) / 1024 * 1024;
    }
};

// 8-byte entries before the 4-byte area: header, every layer, the lm_head partials (2 per workgroup, padded to 4 KB).
inline uint64_t exchange_entries64(int layers, const Shape& s) {
    const XLayout X(s.heads, s.kv_heads, s.hidden, s.inter, s.blocks);
    return uint64_t(kHdrEntries) + uint64_t(layers) * uint64_t(X.per_layer64) + (2ull * s.blocks + 511) / 512 * 512;
}

// The stage-timing build (compiled with LRM_PERSIST_STAMPS): per workgroup 64 constant-clock stamps after the
// exchange entries. Stamps k < 16 and 16 + k: stage boundary k of layers kStampLayer and kStampLayer + 1; 40 the
// launch start, 41 the end of the layers, 42 the lm_head's x gathered, 43 the lm_head done, 44 (workgroup 0) the step's
// end; 32 + k: thread 0's poll passes in the waits of layer kStampLayer (k: 0 A, 1 B, 2 and 3 C's two parts, 4 D, 5 E);
// 48 + k: thread 0's points inside the stages of layer kStampLayer (kernels_persist.hip, PSUB).
constexpr int kStampLayer = 14, kStampWords = 64;
#if defined(LRM_PERSIST_STAMPS)
constexpr uint64_t kStampEntries = 256ull * kStampWords;
#else
constexpr uint64_t kStampEntries = 0;
#endif

// The whole exchange buffer in 8-byte units.
inline uint64_t exchange_entries(int layers, const Shape& s) {
    const XLayout X(s.heads, s.kv_heads, s.hidden, s.inter, s.blocks);
    return exchange_entries64(layers, s) + (uint64_t(layers) * uint64_t(X.per_layer32) + 1) / 2 + kStampEntries;
}

// nullptr when the instantiated kernel covers the shape, else the reason it does not. The kernel is written for the
// Qwen3-0.6B layer on 256 workgroups (32 per XCD): hidden 1024, 16 query / 8 KV heads of 128, SwiGLU 3072.
inline const char* unsupported(const Shape& s) {
    if (s.head_dim != 128 || s.heads != 16 || s.kv_heads != kXcds) return "16 query / 8 KV heads of 128";
    if (s.blocks != 32 * kXcds) return "256 workgroups";
    if (s.hidden != 1024) return "hidden 1024";
    if (s.inter != 3072) return "SwiGLU width 3072";
    if (s.max_pos % 64) return "max_pos a multiple of 64";
    return nullptr;
}

}  // namespace persist
}  // namespace lrm
