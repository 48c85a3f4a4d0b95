// Workspace of the causal prefill attention (attention_prefill_f16 in kernels_fast.hip), shared by the kernel, its
// contract and the executor that sizes the buffer.
#pragma once

#include <cstdint>

namespace lrm {
namespace attn_prefill {

constexpr int kRows = 32;                   // query rows of a tile
constexpr int kSlotWords = 8192 + 256;      // one partial of a split tile: O^T (2 heads x 64 lanes x 64), then m, l
constexpr int64_t pairs(int64_t rows) { return ((rows + kRows - 1) / kRows) / 2; }
// u32 words: one counter per (KV head, tile pair), padded up to a whole (nonzero) number of 256-byte lines, then
// two partials per pair. The counters must be zero before the first launch; every launch leaves them zero.
constexpr int64_t counter_words(int64_t rows, int64_t kv_heads) { return (kv_heads * pairs(rows) / 64 + 1) * 64; }
constexpr int64_t workspace_words(int64_t rows, int64_t kv_heads) {
    return counter_words(rows, kv_heads) + kv_heads * pairs(rows) * 2 * kSlotWords;
}

}  // namespace attn_prefill
}  // namespace lrm
