// Shapes and exchange layout of the persistent one-sequence decode step (kernels_persist.hip), shared by the kernel,
// its launcher and the executor that sizes its buffers.
#pragma once

#include <cstdint>

namespace lrm {
namespace persist {

constexpr int kWaves = 8, kThreads = 512;
// 256-byte header before the entries: u32 word 0 = launch epoch, 1 = abort, 2 = the stage that aborted, 3 = the bound
// of every wait in 100 MHz constant-clock ticks (0: 0.2 s)
constexpr int kHdrEntries = 32;
constexpr int kVecMax = 4096;    // floats of the LDS vector a stage gathers its input into
// Copies of every vector that all workgroups read (o, x after o_proj, the SwiGLU output, x after down_proj): the
// workgroups of XCD r (blockIdx % 8 = r, the dispatch order) poll copy r, so no copy is polled by more than 1/8 of the
// grid.
constexpr int kReplicas = 8;
// 8-byte entries per (query head, split) attention partial row: (max, sum, out[128]) padded to whole 128-byte lines, so
// one wave writes every line of a row whole (lines written in part by several waves cost a read-modify-write each)
constexpr int kPartStride = 144;

// The one instantiated shape family: per-lane and per-wave work counts of every stage, derived from the model sizes
// and the grid. NCH: 512-wide chunks of the hidden vector per lane; RA: q|k|v rows per wave; NCC: chunks per wave of
// an o_proj row; UD: (gate/up row, chunk) units per wave; NCE: chunks per wave of a down_proj row; KS: waves per
// o_proj / down_proj row.
constexpr int kNCH = 2, kRA = 2, kNCC = 2, kUD = 6, kNCE = 3, kKS = 2;

struct Shape {
    int hidden, heads, kv_heads, head_dim, inter, max_pos, blocks;
};

// The exchange area. 8-byte entries, (tag << 32) | value bits, per layer: the q|k|v projection and the attention
// partials per (query head, split) as (max, sum, out[128]) in rows of kPartStride entries; then the lm_head partials (value, index) per workgroup.
// 4-byte entries per layer, value bits with the lowest mantissa bit replaced by the launch parity, kReplicas copies
// each (copy r at + r * its length): the combined attention output o, x after o_proj, the SwiGLU output, x after
// down_proj. The 4-byte area follows the 8-byte one.
struct XLayout {
    int qkv, part, per_layer;  // 8-byte entries
    int o, x1, a, x2, per_layer32;  // 4-byte entries
#if defined(__HIPCC__)
    __host__ __device__
#endif
    XLayout(int qh, int kvh, int hidden, int inter, int blocks) {
        const int S = blocks / kvh;
        qkv = 0;
        part = (qh + 2 * kvh) * 128;
        per_layer = part + qh * S * kPartStride;
        o = 0;
        x1 = o + kReplicas * qh * 128;
        a = x1 + kReplicas * hidden;
        x2 = a + kReplicas * inter;
        per_layer32 = x2 + kReplicas * hidden;
    }
};

// 8-byte entries before the 4-byte area: header, every layer, the lm_head partials.
inline uint64_t exchange_entries64(int layers, const Shape& s) {
    const XLayout X(s.heads, s.kv_heads, s.hidden, s.inter, s.blocks);
    return uint64_t(kHdrEntries) + uint64_t(layers) * uint64_t(X.per_layer) + 2ull * uint64_t(s.blocks);
}

// The whole exchange buffer in 8-byte units.
inline uint64_t exchange_entries(int layers, const Shape& s) {
    const XLayout X(s.heads, s.kv_heads, s.hidden, s.inter, s.blocks);
    return exchange_entries64(layers, s) + (uint64_t(layers) * uint64_t(X.per_layer32) + 1) / 2;
}

// nullptr when the instantiated kernel covers the shape, else the reason it does not.
inline const char* unsupported(const Shape& s) {
    const int G = s.blocks, W = kWaves;
    if (s.head_dim != 128 || s.heads != 2 * s.kv_heads) return "head_dim 128 and two query heads per KV head";
    if (G < 1 || s.kv_heads < 1 || G % s.kv_heads || G / s.kv_heads > 64) return "workgroups a multiple of kv_heads, at most 64 splits";
    if (s.hidden != 512 * kNCH) return "hidden 1024";
    const int N1 = (s.heads + 2 * s.kv_heads) * 128, QC = s.heads * 128;
    if (N1 > kRA * G * W) return "q|k|v rows at most two per wave";
    if (s.hidden % G || W % (s.hidden / G)) return "hidden rows per workgroup dividing the waves";
    const int KS = W / (s.hidden / G);
    if (KS != kKS) return "waves per o_proj row";
    if (QC != kNCC * KS * 512) return "o_proj chunks per wave";
    if (s.inter % G || 2 * (s.inter / G) * kNCH != kUD * W) return "gate/up units per wave";
    if ((s.hidden / G) * kReplicas > 64 || (s.inter / G) * kReplicas > kThreads) return "rows per workgroup";
    if (s.inter != kNCE * KS * 512) return "down_proj chunks per wave";
    const int items = (s.heads * 16 + G - 1) / G;  // combine items (8 output dims each) per workgroup
    if (QC > kVecMax || s.inter > kVecMax || 2 * G > kVecMax || items * 10 * (G / s.kv_heads) > kVecMax)
        return "vector sizes";
    if (items > W) return "combine items";
    if (s.max_pos % 64) return "max_pos a multiple of 64";
    return nullptr;
}

}  // namespace persist
}  // namespace lrm
